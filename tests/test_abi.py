"""The C-ABI library loads on the host and exports every entry point the header declares."""
import ctypes
import os
import re

from hackthenorth_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "htn_decode.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(?:int|int64_t)\s+(htn_\w+)\s*\(", text)))


def declared_arity():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(?:int|int64_t)\s+(htn_\w+)\s*\(([^)]*)\)", text):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_header_and_binding_agree():
    names = declared()
    assert names, "no entry points parsed from the header"
    assert sorted(_lib.SIGNATURES) == names
    arity = declared_arity()
    for name, args in _lib.SIGNATURES.items():
        assert len(args) == arity[name], name


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.htn_version() == 1


def test_argument_errors_are_reported_without_a_gpu():
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    # Null pointers and bad sizes are rejected before any launch.
    assert lib.htn_gemv(null, null, null, 16, 16, null) == _lib.HTN_EINVAL
    assert lib.htn_rms_norm(null, 16, null, null, 1, 16, 1e-6, null) == _lib.HTN_EINVAL
    assert lib.htn_embed_gather(None, 1, null, 10, 8, null, null) == _lib.HTN_EINVAL
    assert lib.htn_attention_scratch_bytes(1, 16, 1, 575) > 0
    assert lib.htn_attention_scratch_bytes(0, 16, 1, 575) == 0
    # The tiled GEMM's k split: partials for a short prompt's long-K
    # projection, none for a full grid, none for k off the 64-wide steps.
    assert lib.htn_gemm_tiles_scratch_bytes(256, 4096, 12288, _lib.EPI_RESIDUAL) > 0
    assert lib.htn_gemm_tiles_scratch_bytes(2048, 4096, 12288, _lib.EPI_RESIDUAL) == 0
    assert lib.htn_gemm_tiles_scratch_bytes(256, 4096, 12290, _lib.EPI_RESIDUAL) == 0
    assert lib.htn_gemm_tiles(null, 4096, null, 16, 64, 8, 0, null, 0, null, 16, null,
                              null) == _lib.HTN_EINVAL
    # Checked before any launch: k off the 64-wide steps, a misaligned scratch.
    p = ctypes.c_void_p(4096)
    assert lib.htn_gemm_tiles(p, 128, p, 16, 100, 8, 0, null, 0, p, 16, null,
                              null) == _lib.HTN_EUNSUPPORTED
    assert lib.htn_gemm_tiles(p, 128, p, 16, 128, 8, 0, null, 0, p, 16, ctypes.c_void_p(4104),
                              null) == _lib.HTN_EUNSUPPORTED
    # 8-bit GEMVs reject unknown formats and missing scales.
    one = ctypes.c_void_p(256)
    assert lib.htn_gemv_w8(one, one, one, 3, one, 16, 16, null) == _lib.HTN_EINVAL
    assert lib.htn_gemv_w8(one, one, null, 1, one, 16, 16, null) == _lib.HTN_EINVAL
    assert lib.htn_fill_weights_w8(one, 16, 0, 0, 0, null) == _lib.HTN_EINVAL


def test_header_constants_match_the_binding():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (HTN_\w+) \(?(-?\d+)\)?", text))
    assert int(consts["HTN_HEAD_SCRATCH_BYTES"]) == _lib.HEAD_SCRATCH_BYTES
    assert int(consts["HTN_ATTENTION_XCD_MISMATCH_BYTE"]) == _lib.ATTENTION_XCD_MISMATCH_BYTE
    assert int(consts["HTN_ATTENTION_OUTPUT_ERROR_BYTE"]) == _lib.ATTENTION_OUTPUT_ERROR_BYTE
    assert int(consts["HTN_ATTENTION_OUTPUT_ACC_BYTE"]) == _lib.ATTENTION_OUTPUT_ACC_BYTE
    assert int(consts["HTN_EINVAL"]) == _lib.HTN_EINVAL
    assert int(consts["HTN_HEAD_DIM"]) == _lib.HEAD_DIM
