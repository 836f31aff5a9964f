"""Fixed-address KV storage and a graph-captured single-token decode step.

Mirrors dryft/engine/decode.py: KVCache (25-46), RotaryTable (49-67),
forward (78-99), DecodeState (102-206) and stream_decode (8-22), with the
same device-resident token/position state so a captured step replays
without host involvement. The batch-one step is five HIP kernels per layer:

  gemv_norm(ln1, W_qkv) -> decode attention with the output projection
  (QK-norm, RoPE from the step's row, KV append, split-KV softmax; each kv
  head's XCD merges its heads and multiplies their columns of W_o) -> the
  partials' sum + residual -> gemv_norm_swiglu(ln2, W_gate_up) ->
  gemv_residual(W_down)

plus one embedding gather before the layers and one fused
final-norm/LM-head/argmax kernel after them, which also writes the token and
advances the position.
"""
import torch

from ._lib import HEAD_DIM
from .kernels.attention import (check_xcd_merge, decode_attention, grouped_attention,
                                prologue_attention, prologue_attention_output)
from .kernels.down import down_residual
from .kernels.embed import embed_gather, embed_gather_pair
from .kernels.fused import norm_rope_cache
from .kernels.greedy import greedy_head
from .kernels.projection import norm_projection, output_projection_residual
from .kernels.rows import (TILE_ROWS, greedy_rows, projection_rows, residual_norm_rows,
                           residual_rows, splits_k, swiglu_rows)
from .speculate import draft_width, verified_tokens


def stream_decode(state, first_tokens, output_length):
    """Launch the next step before yielding the current tokens (decode.py:8-22).

    Only the Python list crosses the yield; output_length=1 launches nothing.
    """
    tokens = first_tokens
    for step in range(output_length):
        has_next = step + 1 < output_length
        if has_next:
            state.graph.replay()
        yield tokens
        if has_next:
            tokens = state.token[:, 0].tolist()


class KVCache:
    """Per-layer K and V of shape [B, Hkv, capacity, 128], zero-filled, in one allocation."""

    def __init__(self, model, batch_size, capacity):
        c = model.config
        shape = (c.num_hidden_layers, 2, batch_size, c.num_key_value_heads, capacity, c.head_dim)
        # Masked slots must still be finite: the zero fill keeps them so.
        self.storage = torch.zeros(shape, dtype=model.dtype, device=model.device)
        self.keys = [self.storage[i, 0] for i in range(c.num_hidden_layers)]
        self.values = [self.storage[i, 1] for i in range(c.num_hidden_layers)]
        self.capacity = capacity
        self.prefill = True


def rope_tables(config, capacity):
    """Default RoPE rows for positions 0..capacity-1, computed like the model's
    rotary module (fp32 inverse frequencies and angles, cos/sin rounded to bf16)."""
    d = config.head_dim
    inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    angles = torch.arange(capacity, dtype=torch.int64).float()[:, None] * inv_freq[None, :]
    emb = torch.cat((angles, angles), dim=-1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


class RotaryTable:
    """Prompt-independent RoPE rows for every cache slot, resident on the device.

    `tables` is (cos, sin), each [1, capacity, 128], as the reference's table
    (decode.py:55-62); `select` gathers rows by device positions. `rows` holds
    the same values as one [capacity, 256] table (cos | sin per slot), so the
    decode step gathers its row with a single launch and every layer's
    attention reads it at a fixed address.
    """

    def __init__(self, model, capacity, enabled=True):
        cos, sin = rope_tables(model.config, capacity)
        self.tables = (cos[None].to(model.device), sin[None].to(model.device))
        self.rows = torch.cat((cos, sin), dim=-1).to(model.device).contiguous()

    def step_row(self, position):
        """(cos, sin) rows [1, 128] for the device position, one gather launch."""
        row = embed_gather(position.reshape(1), self.rows)
        return row[:, :HEAD_DIM], row[:, HEAD_DIM:]

    def select(self, positions):
        """(cos, sin) rows [1, T, 128] for device positions; a position outside
        the table gives zero rows (the gather kernel checks every id)."""
        return tuple(embed_gather(positions.reshape(-1), t[0]).unsqueeze(0) for t in self.tables)


def decode_layer(model, i, h, cache, position, rotary, rope=None):
    """Decoder layer i for one token at batch one: five kernels, h [1, H] -> [1, H].

    Appends the layer's K/V at the device `position`. `rope`, the step's
    (cos, sin) rows from RotaryTable.step_row, lets the attention kernel load
    them without waiting for the position; without it the kernel looks the
    row up in the rotary table by position.
    """
    c = model.config
    layer = model.layers[i]
    groups = c.num_attention_heads // c.num_key_value_heads
    q_width, k_width, _ = c.widths
    cos, sin = rotary.tables
    ln1, ln2 = layer.input_layernorm, layer.post_attention_layernorm
    packed = norm_projection(h, ln1.weight, layer.qkv_weight, ln1.variance_epsilon)
    if rope is not None:
        # Attention and the output projection with its residual in one call.
        r = prologue_attention_output(packed, layer.q_norm, layer.k_norm, rope[0], rope[1],
                                      cache.keys[i], cache.values[i], position,
                                      c.num_key_value_heads, groups, q_width,
                                      q_width + k_width, layer.o_weight, h)
    else:
        a = decode_attention(packed, layer.q_norm, layer.k_norm, cos[0], sin[0],
                             cache.keys[i], cache.values[i], position,
                             c.num_key_value_heads, groups, q_width, q_width + k_width)
        r = output_projection_residual(a, layer.o_weight, h)
    m = norm_projection(r, ln2.weight, layer.gate_up_weight, ln2.variance_epsilon,
                        swiglu=True)
    return down_residual(m, layer.down_weight, r)


def _decode_one(model, token_ids, cache, position, rotary, out=None, advance=None, record=None):
    """Batch-one single-token step through the fused kernels.

    `record`, when a list, receives the hidden state after every layer."""
    # The token's embedding row and the step's RoPE row: one gather launch.
    h, row = embed_gather_pair(token_ids.reshape(1), model.embed_weight, position.reshape(1),
                               rotary.rows)
    rope = (row[:, :HEAD_DIM], row[:, HEAD_DIM:])
    for i in range(len(model.layers)):
        h = decode_layer(model, i, h, cache, position, rotary, rope)
        if record is not None:
            record.append(h)
    if out is None:
        out = torch.empty((1, 1), dtype=torch.int64, device=model.device)
    greedy_head(h, model.norm.weight, model.norm.variance_epsilon, model.lm_head_weight,
                out, advance)
    return out


def _attention_chunks(q, keys, values, positions, groups):
    """grouped_attention over the T queries, written token-major: returns
    [B * T, Hq * 128] rows for the output projection, no transpose. More than
    8 queries (a prefill) go to the causal kernel in one launch; up to 8 (a
    verify pass) in chunks the split kernel takes at once (at most 8 queries
    and 32 query rows per kv head)."""
    b, heads, t, dim = q.shape
    out = torch.empty((b, t, heads, dim), dtype=q.dtype, device=q.device)
    if t > 8:
        grouped_attention(q, keys, values, positions, out=out.transpose(1, 2))
        return out.view(b * t, heads * dim)
    step = max(1, min(8, 32 // groups))
    for s in range(0, t, step):
        e = min(t, s + step)
        grouped_attention(q[:, :, s:e], keys, values, positions[s:e],
                          out=out[:, s:e].transpose(1, 2))
    return out.view(b * t, heads * dim)


def _forward_rows(model, token_ids, cache, positions, last_only, position_embeddings, rotary,
                  record=None):
    """Any batch and token count (prefill, verify): multi-row MFMA projections
    that read each weight once per 32 rows, batched norm/RoPE/cache append and
    grouped attention. 8-bit weights take the batch-one GEMVs row by row.
    `record`, when a list, receives every layer's output rows [B, T, H]."""
    c = model.config
    b, t = token_ids.shape
    hidden = c.hidden_size
    if position_embeddings is None:
        position_embeddings = rotary.select(positions)
    cos, sin = position_embeddings
    h = embed_gather(token_ids, model.embed_weight).reshape(b * t, hidden)
    widths = c.widths
    groups = c.num_attention_heads // c.num_key_value_heads
    rows = b * t
    multi = not c.quantized
    hn = None  # the down projection's output normalised for the next layer (multi-row path)
    for i, layer in enumerate(model.layers):
        ln1, ln2 = layer.input_layernorm, layer.post_attention_layernorm
        if multi and hn is not None:
            packed = projection_rows(hn, layer.qkv_weight)
        elif multi:
            packed = projection_rows(h, layer.qkv_weight, ln1.weight, ln1.variance_epsilon)
        else:
            packed = torch.stack([norm_projection(h[r], ln1.weight, layer.qkv_weight,
                                                  ln1.variance_epsilon) for r in range(rows)])
        if t == 1 and positions.numel() == 1:
            # One token per sequence at one shared position (batched decode):
            # QK-norm, RoPE and the K/V append inside the attention launch,
            # with norm_rope_cache's per-head arithmetic (bit-identical).
            a = prologue_attention(packed.view(b, 1, -1), layer.q_norm, layer.k_norm, cos, sin,
                                   cache.keys[i], cache.values[i], positions,
                                   c.num_key_value_heads, groups, widths[0],
                                   widths[0] + widths[1]).view(b, -1)
        else:
            q, k, v = packed.view(b, t, -1).split(widths, -1)
            shape = (b, t, -1, c.head_dim)
            q, _, _ = norm_rope_cache(q.view(shape), k.view(shape), v.view(shape), layer.q_norm,
                                      layer.k_norm, cos, sin, cache.keys[i], cache.values[i],
                                      positions)
            a = _attention_chunks(q, cache.keys[i], cache.values[i], positions, groups)
        if multi:
            # A projection that splits K writes the next RMSNorm in its split
            # finish, and a prompt's projections (TILE_ROWS rows or more) write
            # it with their residual add; otherwise the next projection
            # normalises its rows itself.
            if rows >= TILE_ROWS or splits_k(*layer.o_weight.shape, rows):
                r, rn = residual_norm_rows(a, layer.o_weight, h, ln2.weight,
                                           ln2.variance_epsilon)
                m = swiglu_rows(rn, layer.gate_up_weight)
            else:
                r = residual_rows(a, layer.o_weight, h)
                m = swiglu_rows(r, layer.gate_up_weight, ln2.weight, ln2.variance_epsilon)
            nxt = model.layers[i + 1].input_layernorm if i + 1 < len(model.layers) \
                else model.norm
            if rows >= TILE_ROWS or splits_k(*layer.down_weight.shape, rows):
                h, hn = residual_norm_rows(m, layer.down_weight, r, nxt.weight,
                                           nxt.variance_epsilon)
            else:
                h, hn = residual_rows(m, layer.down_weight, r), None
        else:
            r = torch.stack([output_projection_residual(a[j], layer.o_weight, h[j])
                             for j in range(rows)])
            m = torch.stack([norm_projection(r[j], ln2.weight, layer.gate_up_weight,
                                             ln2.variance_epsilon, swiglu=True)
                             for j in range(rows)])
            h = torch.stack([down_residual(m[j], layer.down_weight, r[j]) for j in range(rows)])
        if record is not None:
            record.append(h.view(b, t, hidden))
    kept = 1 if last_only else t
    if multi:
        if hn is not None:
            # hn is the final RMSNorm of h (the last down projection fused it).
            xn = hn.view(b, t, hidden)
            xn = xn[:, -1:] if last_only else xn
            return greedy_rows(xn.reshape(-1, hidden).contiguous(),
                               model.lm_head_weight).view(b, kept)
        x = h.view(b, t, hidden)
        x = x[:, -1:] if last_only else x
        return greedy_rows(x.reshape(-1, hidden).contiguous(), model.lm_head_weight,
                           model.norm.weight, model.norm.variance_epsilon).view(b, kept)
    x = h.view(b, t, hidden)
    flat = (x[:, -1:] if last_only else x).reshape(-1, hidden).contiguous()
    out = torch.empty((flat.shape[0],), dtype=torch.int64, device=model.device)
    for r in range(flat.shape[0]):
        greedy_head(flat[r], model.norm.weight, model.norm.variance_epsilon,
                    model.lm_head_weight, out[r:r + 1])
    return out.view(b, kept)


def forward(model, token_ids, cache, positions, attention_mask=None, last_only=True,
            position_embeddings=None, *, rotary=None, out=None, advance=None, record=None):
    """Greedy next tokens [B, 1] (or [B, T] with last_only=False) (decode.py:78-99).

    Causality comes from the absolute `positions` (device int64, one per
    token) inside the attention kernels, so `attention_mask` is accepted and
    ignored, as in the reference's position-causal attention. K/V of the new
    tokens are written to cache slots `positions`. With a RotaryTable and a
    single token at batch one the fused step runs; `out`/`advance` then
    receive the token and a position increment in place. `record` (a list)
    collects the per-layer hidden states on either path.
    """
    b, t = token_ids.shape
    if b == 1 and t == 1 and rotary is not None and position_embeddings is None:
        return _decode_one(model, token_ids, cache, positions, rotary, out, advance, record)
    if rotary is None and position_embeddings is None:
        rotary = RotaryTable(model, cache.capacity)
    tokens = _forward_rows(model, token_ids, cache, positions, last_only, position_embeddings,
                           rotary, record)
    if out is not None:
        out.copy_(tokens[:, -1:])
    if advance is not None:
        advance.add_(t)
    return tokens


class DecodeState:
    """Cache, rotary table, device token/position and the captured step (decode.py:102-206)."""

    def __init__(self, model, batch_size, prompt_length, output_length, speculative=False,
                 cache_rotary=True, omit_unused_masks=True, draft_tokens=None):
        self.shape = (batch_size, prompt_length, output_length)
        self.draft_tokens = draft_width(output_length) if speculative and batch_size == 1 else 0
        if speculative and batch_size == 1 and draft_tokens is not None:
            self.draft_tokens = int(draft_tokens)  # a draft model's fixed proposal width
        # Tail verification may write beyond the last requested output; causal
        # attention hides those scratch slots from earlier queries.
        capacity = prompt_length + output_length - 1 + self.draft_tokens
        if self.draft_tokens:
            # The verifier is captured at the prompt length: its k + 1 rows
            # need slots there even for a one-token request.
            capacity = max(capacity, prompt_length + self.draft_tokens + 1)
        device = model.device
        self.model = model
        self.capacity = capacity
        self.cache = KVCache(model, batch_size, capacity)
        self.prompt_positions = torch.arange(prompt_length, device=device)
        self.token = torch.zeros((batch_size, 1), dtype=torch.int64, device=device)
        self.position = torch.full((1,), prompt_length, dtype=torch.int64, device=device)
        self.rotary = RotaryTable(model, capacity, enabled=cache_rotary)
        self.graph = None
        self.verify_graph = None
        if output_length > 1:
            self.capture(model)
        if self.draft_tokens > 0:
            self.capture_verifier(model)

    def step(self, model):
        forward(model, self.token, self.cache, self.position, rotary=self.rotary,
                out=self.token, advance=self.position)

    def check_merge(self):
        """Raise if an in-kernel attention merge of this device saw a split on
        another XCD (kernels.attention.check_xcd_merge); synchronises."""
        check_xcd_merge(self.model.device)

    def capture(self, model):
        self.cache.prefill = False
        prompt_length = self.shape[1]
        stream = torch.cuda.Stream(device=model.device)
        stream.wait_stream(torch.cuda.current_stream(model.device))
        # Captures always run in inference mode: torch keeps per-generator
        # graph state tensors shared by every live graph, created in the mode
        # of the capture that made them; capturing in inference mode can
        # update them whichever mode made them.
        with torch.inference_mode(), torch.cuda.stream(stream):
            # Library load and allocator warm-up happen off capture.
            for _ in range(2):
                self.position.fill_(prompt_length)
                self.step(model)
            self.position.fill_(prompt_length)
        torch.cuda.current_stream(model.device).wait_stream(stream)
        self.graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(self.graph, stream=stream):
            self.step(model)

    def prefill(self, model, input_ids):
        """The whole prompt in one causal multi-row pass (decode.py:157-166).

        Every prompt token's K/V goes to its cache slot, the projections read
        each weight once per 32 rows, attention is causal by absolute position,
        and only the last row of each sequence reaches the LM head. Afterwards
        `token` holds the greedy continuation and `position` equals the prompt
        length. Launches only: it can be captured (prefill.prefill does).
        """
        batch, length = input_ids.shape
        if (batch, length) != self.shape[:2]:
            raise ValueError("prompt shape differs from the state's shape")
        self.cache.prefill = True
        token = forward(model, input_ids, self.cache, self.prompt_positions, rotary=self.rotary)
        self.cache.prefill = False
        self.token.copy_(token)
        self.position.fill_(length)
        return self.token

    def prefill_stepwise(self, model, input_ids):
        """The prompt through the captured decode step one token at a time (each
        replay attends over the slots written so far): the same causal prefill
        computed token by token, kept as a cross-check of the batched pass."""
        batch, length = input_ids.shape
        if (batch, length) != self.shape[:2] or batch != 1:
            raise ValueError("stepwise prefill takes one prompt of the state's length")
        self.cache.prefill = False
        self.position.fill_(0)
        for i in range(length):
            self.token.copy_(input_ids[:, i:i + 1])
            if self.graph is not None:
                self.graph.replay()
            else:
                self.step(model)
        return self.token

    def verify_step(self, model):
        """Forward of the verify input at positions position .. position + k
        (decode.py:168-179): every row's greedy token, multi-row projections."""
        positions = self.position + self.verify_offsets
        return forward(model, self.verify_input, self.cache, positions, last_only=False,
                       rotary=self.rotary)

    def capture_verifier(self, model):
        """Capture verify_step as a graph over a fixed-address input (decode.py:181-195)."""
        length = self.draft_tokens + 1
        device = model.device
        self.verify_input = torch.zeros((1, length), dtype=torch.int64, device=device)
        self.verify_offsets = torch.arange(length, device=device)
        prompt_length = self.shape[1]
        self.position.fill_(prompt_length)
        stream = torch.cuda.Stream(device=device)
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.inference_mode(), torch.cuda.stream(stream):
            for _ in range(2):
                self.verify_step(model)
        torch.cuda.current_stream(device).wait_stream(stream)
        self.verify_graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(self.verify_graph, stream=stream):
            self.verify_output = self.verify_step(model)
        self.position.fill_(prompt_length)

    def verify(self, current_token, proposal, position):
        """Score [current, *proposal] at positions position.. in one pass and keep
        the verified prefix plus one target token (decode.py:197-206). A
        proposal of the captured width replays the verify graph."""
        inputs = torch.tensor([[current_token, *proposal]], dtype=torch.int64,
                              device=self.token.device)
        if self.verify_graph is not None and inputs.shape[1] == self.verify_input.shape[1]:
            self.verify_input.copy_(inputs)
            self.position.fill_(position)
            self.verify_graph.replay()
            predictions = self.verify_output
        else:
            positions = torch.arange(position, position + inputs.shape[1],
                                     device=self.token.device)
            predictions = forward(self.model, inputs, self.cache, positions, last_only=False,
                                  rotary=self.rotary)
        emitted = verified_tokens(proposal, predictions[0].tolist())
        self.token.copy_(predictions[:, len(emitted) - 1:len(emitted)])
        # The speculative tail is discarded logically: later queries mask it and
        # later steps overwrite those slots.
        self.position.fill_(position + len(emitted))
        return emitted
