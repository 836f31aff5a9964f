"""Weight-only 8-bit projection weights (int8 or fp8 e4m3fn, per-row fp32 scale).

The reference decodes in bf16 only; this adds the 8-bit storage the decode
GEMVs can stream at half the bytes. A QuantizedWeight stands wherever a bf16
[N, K] projection weight is accepted (norm_projection, output_projection_residual,
down_residual, projection, greedy_head): the ops dispatch on its type, so the
decode layer code is the same for every format.

  y[n] = bf16(scale[n] * sum_k x[k] * w[n, k])   (fp32 accumulation)

int8 weights are two's complement; fp8 weights are OCP e4m3fn (bias 7, max
448, codes 0x7f/0xff are NaN). Both are held as raw bytes (torch.uint8).
"""
import torch

from . import _lib

FORMATS = {"int8": 1, "fp8_e4m3": 2}


class QuantizedWeight:
    """Row-major 8-bit weight bytes [N, K] plus one fp32 scale per row."""

    def __init__(self, data, scale, fmt):
        if fmt not in FORMATS:
            raise ValueError(f"unknown weight format {fmt!r}; expected one of {sorted(FORMATS)}")
        if data.dtype != torch.uint8 or data.dim() != 2 or not data.is_contiguous():
            raise ValueError("quantized weight bytes must be a contiguous uint8 [N, K] tensor")
        if scale.dtype != torch.float32 or scale.shape != (data.shape[0],):
            raise ValueError("scales must be float32 with one value per weight row")
        self.data = data
        self.scale = scale.contiguous()
        self.format = fmt

    @property
    def code(self):
        return FORMATS[self.format]

    @property
    def shape(self):
        return self.data.shape

    @property
    def device(self):
        return self.data.device

    def is_contiguous(self):
        return True

    def numel(self):
        return self.data.numel()

    def nbytes(self):
        """Bytes a GEMV streams: one per weight plus four per row scale."""
        return self.data.numel() + 4 * self.scale.numel()

    @classmethod
    def empty(cls, rows, cols, fmt, device):
        return cls(torch.empty((rows, cols), dtype=torch.uint8, device=device),
                   torch.empty((rows,), dtype=torch.float32, device=device), fmt)

    @classmethod
    def quantize(cls, w, fmt):
        """Symmetric per-row quantization of a [N, K] weight (checkpoint loading,
        not the decode path): scale = max|w_n| / qmax with qmax 127 (int8) or
        448 (fp8), codes = round-to-nearest-even(w / scale)."""
        if fmt not in FORMATS:
            raise ValueError(f"unknown weight format {fmt!r}")
        wf = w.float()
        qmax = 127.0 if fmt == "int8" else 448.0
        scale = wf.abs().amax(dim=1).clamp_min(1e-30) / qmax
        v = wf / scale[:, None]
        if fmt == "int8":
            codes = torch.round(v).clamp_(-127, 127).to(torch.int8).view(torch.uint8)
        else:
            codes = v.clamp_(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        return cls(codes.contiguous(), scale.contiguous(), fmt)

    def randomize_(self, seed, stream, scale_stream, scale_lo=0.001, scale_hi=0.01):
        """Uniform integer weights in [-127, 127] (fp8: their RNE e4m3fn codes) and
        scales U(scale_lo, scale_hi), from the seeded device generator."""
        _lib.require_gpu(self.data)
        st = _lib.stream(self.device)
        _lib.call("htn_fill_weights_w8", _lib.ptr(self.data), self.data.numel(), seed, stream,
                  self.code, st)
        span = float(torch.tensor(scale_hi - scale_lo, dtype=torch.float32))
        _lib.call("htn_fill_uniform_f32", _lib.ptr(self.scale), self.scale.numel(), seed,
                  scale_stream, float(scale_lo), span, st)
        return self
