"""Captured prefill for prompts of up to 2048 tokens (dryft/engine/prefill.py:6-26).

The first prefill of a DecodeState records its batched prompt pass
(DecodeState.prefill: one multi-row causal forward, last row to the LM head)
into a HIP graph over a fixed-address input; later prompts of the same shape
copy their ids in and replay it. The graph rewrites every prompt KV slot and
resets the token and position, so replays need no other reset. Longer prompts
run the pass eagerly: they keep the GPU busy without a graph.
"""
import torch

GRAPH_LIMIT = 2048


def prefill(model, state, input_ids):
    """Prefill `input_ids` [B, P] into `state`; returns state.token ([B, 1])."""
    if input_ids.numel() > GRAPH_LIMIT:
        return state.prefill(model, input_ids)
    if getattr(state, "prefill_graph", None) is None:
        device = model.device
        state.prefill_input = torch.empty_like(input_ids)
        state.prefill_input.copy_(input_ids)
        stream = torch.cuda.Stream(device=device)
        stream.wait_stream(torch.cuda.current_stream(device))
        # Warm-up off capture (library load, scratch sizing), then the capture;
        # in inference mode, as every capture of this package.
        with torch.inference_mode(), torch.cuda.stream(stream):
            for _ in range(2):
                state.prefill(model, state.prefill_input)
        torch.cuda.current_stream(device).wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(graph, stream=stream):
            state.prefill(model, state.prefill_input)
        state.prefill_graph = graph
    else:
        state.prefill_input.copy_(input_ids)
    state.prefill_graph.replay()
    return state.token
