"""The output projection fused into the decode attention launch
(htn_prologue_attention_output) against the two separate steps it replaces:
prologue_attention (dryft/engine/kernels/attention.py:162) then
output_projection_residual (dryft/engine/kernels/projection.py:70).

The fused projection sums the same fp32 products in another order (each kv
head's columns in fp32, then the head groups exactly, in 64-bit fixed
point), so its rounded sum may differ by one bf16 ulp of the sum and, after
the residual add, by one ulp of the output: every element must be within
ulp(sum) + ulp(out) of the unfused result, with the sum taken in float64 on
the CPU from the attention rows. The cache append is bit-identical. Repeated calls,
calls at shrinking and growing contexts, and graph replays check that the
per-pair flags it uses are left armed for the next call; the scratch's error
and mismatch words stay zero. Projections under 16 MB take the unfused path
(the library's count of fused calls tells which path ran).
"""
import pytest
import torch

from oracle import qwen3 as Q
from oracle import rng as ORNG
from hackthenorth_amd.kernels import attention as A
from hackthenorth_amd.kernels.projection import output_projection_residual
from hackthenorth_amd.model import Norm
from hackthenorth_amd.quant import QuantizedWeight

pytestmark = pytest.mark.gpu


def nrm(stream, shape, std=1.0, seed=13):
    return Q.normal_bf16(seed, stream, shape, std).to("cuda")


def ulp(v):
    return torch.pow(2.0, torch.floor(torch.log2(v.double().abs().clamp_min(1e-30))) - 7)


def unfused(packed, qg, kg, cos, sin, keys, values, pos, kv, groups, width, w, h):
    a = A.prologue_attention(packed, qg, kg, cos, sin, keys, values, pos, kv, groups, width,
                             width + kv * 128)
    return a, output_projection_residual(a.view(1, -1), w, h)


def case(width, kv, n, cap, fmt, seed):
    heads = width // 128
    qg, kg = Norm(nrm(1, (128,), seed=seed), 1e-6), Norm(nrm(2, (128,), seed=seed), 1e-6)
    cos_t, sin_t = Q.rope_tables(cap, 128, 1e6)
    packed = nrm(3, (1, 1, width + 2 * kv * 128), seed=seed)
    keys, values = nrm(4, (1, kv, cap, 128), seed=seed), nrm(5, (1, kv, cap, 128), seed=seed)
    w = nrm(6, (n, width), std=0.02, seed=seed)
    if fmt != "bf16":
        w = QuantizedWeight.quantize(w, fmt)
    h = nrm(7, (1, n), seed=seed)
    return dict(heads=heads, qg=qg, kg=kg, cos_t=cos_t, sin_t=sin_t, packed=packed, keys=keys,
                values=values, w=w, h=h)


def accumulators(width, n, cap):
    """The fused projection's 64-bit row accumulators [n] in the current
    stream's attention scratch (inside its leading zero region, which every
    call leaves zero)."""
    from hackthenorth_amd import _lib
    lib = _lib.load()
    nbytes = lib.htn_attention_output_scratch_bytes(1, width // 128, width // 128, cap, n)
    # The buffer the call will use (kept per stream, grown to this size).
    buf = A._scratch(torch.device("cuda"), 1, width // 128, 1, cap, nbytes)
    off = _lib.ATTENTION_OUTPUT_ACC_BYTE
    return buf.view(torch.uint8)[off:off + n * 8].view(torch.int64)


def check_one(c, width, kv, n, p, label, fused):
    cos = c["cos_t"][p:p + 1][None].to("cuda")
    sin = c["sin_t"][p:p + 1][None].to("cuda")
    pos = torch.tensor([p], dtype=torch.int64, device="cuda")
    k1, v1 = c["keys"].clone(), c["values"].clone()
    k2, v2 = c["keys"].clone(), c["values"].clone()
    groups = c["heads"] // kv
    a, ref = unfused(c["packed"], c["qg"], c["kg"], cos, sin, k1, v1, pos, kv, groups, width,
                     c["w"], c["h"])
    from hackthenorth_amd import _lib
    acc = accumulators(width, n, c["keys"].shape[2])
    before = _lib.load().htn_attention_output_fused_calls()
    got = A.prologue_attention_output(c["packed"], c["qg"], c["kg"], cos, sin, k2, v2, pos, kv,
                                      groups, width, width + kv * 128, c["w"], c["h"])
    assert _lib.load().htn_attention_output_fused_calls() - before == int(fused), label
    # Every row completed: the accumulators are clear for the next call.
    assert int(acc.abs().max()) == 0, label
    assert torch.equal(k1, k2) and torch.equal(v1, v2), label
    w = c["w"]
    x = a.view(-1).cpu().double()
    if not isinstance(w, QuantizedWeight):
        total = w.cpu().double() @ x
    else:
        codes = w.data.cpu().numpy().reshape(-1)
        vals = torch.from_numpy(ORNG.w8_values(codes, w.format)).view(n, width).double()
        total = (vals @ x) * w.scale.cpu().double()
    bound = ulp(total) + ulp(ref.view(-1).cpu().float())
    diff = (got.view(-1).cpu().double() - ref.view(-1).cpu().double()).abs()
    worst = float((diff / bound).max())
    print(f"{label}: {int((diff > 0).sum())} of {n} differ, worst {worst:.3g} of the bound",
          flush=True)
    assert bool((diff <= bound).all()), label
    return got


@pytest.mark.parametrize("width,kv,n,cap,positions,fmt,fused", [
    (4096, 8, 4096, 2304, (2047, 2100, 2047), "bf16", True),     # 8B, context 2048
    (4096, 8, 4096, 8320, (8191, 8200), "int8", True),           # 8B 8-bit at 8K
    (4096, 8, 4096, 8320, (8191,), "fp8_e4m3", True),
    (4096, 8, 2560, 4100, (4095,), "bf16", True),                # 4B, context 4096
    (1024, 2, 8192, 300, (7, 299), "bf16", True),                # two kv heads, 8192 rows
    # Projections under 16 MB stay unfused (the 0.6B shape, tiny widths).
    (2048, 8, 1024, 576, (511, 540, 575), "bf16", False),
    (512, 2, 256, 300, (7, 299), "bf16", False),
    (4096, 8, 4096, 60, (5, 59), "bf16", False),                 # one split: unfused
    (4096, 8, 4096, 12000, (11999,), "bf16", False),             # > 24 splits: unfused
])
def test_fused_output_projection_matches_separate_steps(width, kv, n, cap, positions, fmt, fused):
    A.xcd_merge_mismatches(reset=True)
    c = case(width, kv, n, cap, fmt, seed=width + cap)
    with torch.inference_mode():
        for rep in range(2):
            for p in positions:
                check_one(c, width, kv, n, p, f"width {width} n {n} {fmt} pos {p} rep {rep}",
                          fused)
    assert A.xcd_merge_mismatches() == 0


def test_fused_output_projection_in_a_graph_replays_exactly():
    width, kv, n, cap, p = 4096, 8, 4096, 2304, 2047
    c = case(width, kv, n, cap, "bf16", seed=5)
    cos = c["cos_t"][p:p + 1][None].to("cuda")
    sin = c["sin_t"][p:p + 1][None].to("cuda")
    pos = torch.tensor([p], dtype=torch.int64, device="cuda")
    groups = c["heads"] // kv
    A.xcd_merge_mismatches(reset=True)

    def call():
        return A.prologue_attention_output(c["packed"], c["qg"], c["kg"], cos, sin, c["keys"],
                                           c["values"], pos, kv, groups, width, width + kv * 128,
                                           c["w"], c["h"])

    with torch.inference_mode():
        eager = call().clone()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            call()
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = call()
        for _ in range(4):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            assert torch.equal(call(), eager)  # eager work between the replays
    assert A.xcd_merge_mismatches() == 0
