"""ctypes binding of libnve_hip.so (the C ABI in include/nve_kernels.h).

Loading fails loudly when the library has not been built: the product path has no
CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libnve_hip.so"

# status / dtype / mode codes (include/nve_kernels.h)
NVE_OK = 0
NVE_ERR_NULL = -1
NVE_ERR_SHAPE = -2
NVE_ERR_ALIGN = -3
NVE_ERR_DTYPE = -4
NVE_ERR_TOO_LARGE = -5
DT_F16, DT_BF16, DT_F32, DT_F32_ACCUM = 0, 1, 2, 3
XS_GROUP32_F32, XS_ROW_BF16 = 0, 1
MAX_K = 32768
GEMV_AUTO, GEMV_ONESHOT, GEMV_PERSISTENT = 0, 1, 2
MAX_M = 16
STAGE_QKV, STAGE_O_MERGE, STAGE_GATE_UP, STAGE_DOWN = 0, 1, 2, 3

_p = C.c_void_p
_i = C.c_int

# name -> (restype, argtypes), every symbol include/nve_kernels.h declares
SIGNATURES: dict[str, tuple] = {
    "nve_quantize_f16_q8": (None, [_p, _p, _p, _i, _p]),
    "nve_matvec_w4a8": (None, [_p, _p, _p, _p, _p, _i, _i, _p]),
    "nve_matvec_w4a16": (None, [_p, _p, _p, _p, _p, _i, _i, _p]),
    "nve_qkv_matvec_w4a16": (None, [_p, _p, _p, _p, _i, _p, _p, _p, _i, _p, _p, _p, _i, _p, _p, _p, _i, _p]),
    "nve_hip_quantize_q8": (_i, [_p, _i, _i, _i, _p, _p, _p]),
    "nve_hip_quantize_q8_rows": (_i, [_p, _i, _i, _i, _p, _p, _p]),
    "nve_hip_matvec_w4a8": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _p]),
    "nve_hip_qkv_matvec_w4a8": (_i, [_p, _p, _p, _p, _i, _p, _p, _i, _p, _p, _i, _p, _p, _p, _i, _i, _p]),
    "nve_hip_grouped_matvec_w4a8": (_i, [_p, _p, _p, _i, _i, _i, _p]),
    "nve_hip_grouped_matvec_w4a16": (_i, [_p, _i, _p, _i, _i, _i, _p]),
    "nve_hip_matvec_w4a8_x": (_i, [_p, _i, _p, _p, _p, _i, _i, _i, _p]),
    "nve_hip_grouped_matvec_w4a8_x": (_i, [_p, _i, _p, _i, _i, _i, _p]),
    "nve_hip_matvec_w4a8_batched": (_i, [_i, _p, _p, _i, _p, _p, _p, _i, _i, _i, _p]),
    "nve_hip_w4a8_block_acc": (_i, [_p, _p, _p, _i, _i, _p]),
    "nve_hip_matvec_w4a16": (_i, [_p, _i, _p, _p, _p, _p, _i, _i, _i, _p]),
    "nve_hip_qkv_matvec_w4a16": (_i, [_p, _i, _p, _p, _p, _i, _p, _p, _p, _i, _p, _p, _p, _i, _p, _p, _p, _i, _i, _p]),
    "nve_hip_q4_quantize": (_i, [_p, _i, _i, _i, _p, _p, _p]),
    "nve_hip_q4_quantize_awq": (_i, [_p, _i, _p, _i, _i, _i, _p, _p, _p, _p]),
    "nve_hip_q4_repack": (_i, [_p, _i, _i, _p, _p, _p]),
    "nve_hip_dequant_w4": (_i, [_p, _p, _p, _p, _i, _i, _i, _p]),
    "nve_hip_gemm_w4a16": (_i, [_p, _i, _i, _p, _p, _p, _p, _i, _i, _i, _p]),
    "nve_hip_gemm_w4a16_workspace_bytes": (C.c_size_t, [_i, _i, _i]),
    "nve_hip_gemm_w4a16_ws": (_i, [_p, _i, _i, _p, _p, _p, _p, _i, _i, _i, _p, C.c_size_t, _p]),
    "nve_dequant_w4a16": (None, [_p, _p, _p, _p, _i, _i, _p]),
    "nve_use_w4a8": (_i, [C.c_double]),
    "nve_hip_stream_read": (_i, [_p, C.c_size_t, _p, _p]),
    "nve_hip_stream_read_mode": (_i, [_p, C.c_size_t, _p, _i, _p]),
    "nve_hip_set_gemv_policy": (_i, [_i, _i, _i]),
    "nve_hip_decode_workspace_bytes": (C.c_size_t, [_p]),
    "nve_hip_layer_forward_decode": (_i, [_p, _p, _p, _i, _p]),
    "nve_hip_layer_forward_decode_noalloc": (_i, [_p, _p, _p, _i, _p]),
    "nve_hip_decode_stage": (_i, [_p, _p, _p, _i, _i, _p, _p, _p]),
    "nve_hip_decode_attn_splits": (_i, [_p]),
    "nve_hip_decode_head": (_i, [_p, _p, _i, _p]),
    "nve_hip_embed": (_i, [_p, _p, _p, _i, _i, _p]),
    "nve_hip_last_status": (_i, []),
    "nve_hip_status_string": (C.c_char_p, [_i]),
    "nve_hip_version": (C.c_char_p, []),
    "nve_hip_build_id": (C.c_char_p, []),
}



class W4Mat(C.Structure):
    """nve_w4_mat (include/nve_kernels.h)."""
    _fields_ = [("nibbles", C.c_void_p), ("scales", C.c_void_p), ("awq", C.c_void_p), ("out", C.c_void_p),
                ("n", C.c_int)]


class DecodeConfig(C.Structure):
    """nve_decode_config."""
    _fields_ = [("hidden", C.c_int), ("num_heads", C.c_int), ("num_kv_heads", C.c_int), ("head_dim", C.c_int),
                ("ffn", C.c_int), ("max_seq", C.c_int), ("vocab", C.c_int), ("eps", C.c_float)]


class W4Weight(C.Structure):
    """nve_w4_weight."""
    _fields_ = [("nibbles", C.c_void_p), ("scales", C.c_void_p), ("n", C.c_int), ("k", C.c_int)]


class LayerWeights(C.Structure):
    """nve_layer_weights."""
    _fields_ = [("input_norm", C.c_void_p), ("post_attn_norm", C.c_void_p)] + [
        (nm, W4Weight) for nm in ("q", "k", "v", "o", "gate", "up", "down")]


class DecodeIO(C.Structure):
    """nve_decode_io."""
    _fields_ = [("hidden", C.c_void_p), ("k_cache", C.c_void_p), ("v_cache", C.c_void_p), ("pos", C.c_void_p),
                ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p), ("workspace", C.c_void_p)]


class DecodeHead(C.Structure):
    """nve_decode_head."""
    _fields_ = [("hidden", C.c_void_p), ("final_norm", C.c_void_p), ("lm_head", W4Weight), ("embed", C.c_void_p),
                ("logits", C.c_void_p), ("token_out", C.c_void_p), ("pos", C.c_void_p), ("workspace", C.c_void_p)]


_lib: C.CDLL | None = None


class NveError(RuntimeError):
    def __init__(self, fn: str, status: int):
        msg = lib().nve_hip_status_string(status).decode()
        super().__init__(f"{fn}: {msg} (status {status})")
        self.status = status


def lib() -> C.CDLL:
    """Load libnve_hip.so (raises if it is missing: there is no fallback path)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        from .build_ext import source_id
        built, tree = L.nve_hip_build_id().decode(), source_id()
        if built != tree:
            raise RuntimeError(
                f"{LIB_PATH} was built from other sources (build id {built}, sources {tree}); "
                "rebuild it: `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        _lib = L
    return _lib


def check(fn: str, status: int) -> None:
    if status != NVE_OK:
        raise NveError(fn, status)
