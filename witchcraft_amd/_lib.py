"""ctypes binding of libt5hip.so (the C ABI in include/t5hip.h).

The library is built in-tree (witchcraft_amd/libt5hip.so).  There is no fallback: if it
is missing or cannot be loaded, importing this module raises.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libt5hip.so"

T5H_OK = 0
T5H_ERR_INVALID = -1
T5H_ERR_FORMAT = -2
T5H_ERR_HIP = -3
T5H_ERR_NOMEM = -4
T5H_ERR_NODEVICE = -5

T5H_NUMERICS_DEFAULT = 0
T5H_NUMERICS_HYBRID = 1
T5H_NUMERICS_HYBRID_BF16 = 2


class T5HConfig(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_int32), ("d_model", C.c_int32), ("d_kv", C.c_int32),
        ("d_ff", C.c_int32), ("num_layers", C.c_int32), ("num_heads", C.c_int32),
        ("relative_attention_num_buckets", C.c_int32),
        ("relative_attention_max_distance", C.c_int32),
        ("layer_norm_epsilon", C.c_float), ("feed_forward_gated", C.c_int32),
        ("proj_dim", C.c_int32), ("max_seq_len", C.c_int32),
    ]


class T5HKernelStat(C.Structure):
    _fields_ = [("name", C.c_char_p), ("launches", C.c_int64), ("total_ms", C.c_double),
                ("flops", C.c_double), ("bytes", C.c_double)]


# Every entry point of include/t5hip.h: name -> (restype, argtypes)
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_vp = C.c_void_p
SIGNATURES = {
    "t5h_last_error": (C.c_char_p, []),
    "t5h_config_xtr_base": (C.c_int, [C.POINTER(T5HConfig)]),
    "t5h_create": (C.c_int, [_u8p, C.c_size_t, C.POINTER(T5HConfig), C.c_int, C.POINTER(C.c_void_p)]),
    "t5h_destroy": (None, [_vp]),
    "t5h_encode": (C.c_int, [_vp, _u32p, _i32p, C.c_int32, _f32p, _vp]),
    "t5h_encode_normalized": (C.c_int, [_vp, _u32p, _i32p, C.c_int32, _f32p, _vp]),
    "t5h_encode_device": (C.c_int, [_vp, _vp, _i32p, C.c_int32, _vp, _vp]),
    "t5h_encode_device_noalloc": (C.c_int, [_vp, _vp, _i32p, C.c_int32, _vp, _vp]),
    "t5h_synchronize": (C.c_int, [_vp]),
    "t5h_stream": (C.c_void_p, [_vp]),
    "t5h_embed_ids": (C.c_int, [_vp, _u32p, C.c_int32, C.c_int32, C.c_int32, _f32p, _i32p,
                                C.POINTER(C.c_int32)]),
    "t5h_embed_batch": (C.c_int, [_vp, _u32p, _i32p, C.c_int32, C.c_int32, C.c_int32, _f32p, _i32p, _i32p]),
    "t5h_quantize_q4k": (C.c_int, [_f32p, C.c_int64, _u8p, C.c_int32]),
    "t5h_set_numerics": (C.c_int, [_vp, C.c_int32]),
    "t5h_q8k_quantize": (C.c_int, [C.c_int32, _f32p, C.c_int32, C.c_int32, _u8p]),
    "t5h_q4k_q8k_matmul": (C.c_int, [C.c_int32, _u8p, C.c_int32, _u8p, C.c_int32, C.c_int32, _f32p]),
    "t5h_q4k_dequant_f32": (C.c_int, [_u8p, C.c_size_t, _f32p, C.c_int]),
    "t5h_attention_work": (C.c_int, [_i32p, C.c_int32, C.c_int32, _i32p, C.c_int32, C.POINTER(C.c_int32)]),
    "t5h_matmul_t": (C.c_int, [C.c_int32, _f32p, C.c_int32, _f32p, C.c_int32, C.c_int32, C.c_int32, _f32p]),
    "t5h_matmul_argmax": (C.c_int, [C.c_int32, _f32p, C.c_int32, _f32p, C.c_int32, C.c_int32, C.c_int32, _u32p]),
    "t5h_matmul_t_device": (C.c_int, [_vp, C.c_int32, _vp, C.c_int32, C.c_int32, C.c_int32, _vp, _vp]),
    "t5h_matmul_argmax_device": (C.c_int, [_vp, C.c_int32, _vp, C.c_int32, C.c_int32, C.c_int32, _vp, _vp]),
    "t5h_q4_dequant_table": (C.c_int, [_f32p]),
    "t5h_q4_compand_thresholds": (C.c_int, [_f32p]),
    "t5h_residual_encode": (C.c_int, [C.c_int32, _f32p, C.c_int32, _f32p, C.c_int32, _u32p, C.c_int32, _u8p]),
    "t5h_residual_encode_device": (C.c_int, [_vp, C.c_int32, _vp, C.c_int32, _vp, C.c_int32, _vp, _vp, _vp]),
    "t5h_residual_decode": (C.c_int, [C.c_int32, _u8p, C.c_int32, C.c_int32, _f32p]),
    "t5h_residual_decode_device": (C.c_int, [_vp, C.c_int32, C.c_int32, _vp, _vp]),
    "t5h_matmul_t_q4": (C.c_int, [C.c_int32, _f32p, C.c_int32, _u8p, C.c_int32, C.c_int32, _f32p]),
    "t5h_matmul_t_q4_device": (C.c_int, [_vp, C.c_int32, _vp, C.c_int32, C.c_int32, _vp, _vp]),
    "t5h_embeddings_to_packed": (C.c_int, [C.c_int32, _f32p, _i32p, C.c_int32, C.c_int32, _u8p, C.c_size_t,
                                           np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS"),
                                           C.POINTER(C.c_double)]),
    "t5h_embeddings_from_packed": (C.c_int, [C.c_int32, _u8p, np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS"),
                                             C.c_int32, C.c_int32, _f32p, C.c_size_t, _i32p,
                                             C.POINTER(C.c_double)]),
    "t5h_layer_forward": (C.c_int, [_vp, C.c_int32, _f32p, _i32p, C.c_int32, _f32p]),
    "t5h_ffn_block": (C.c_int, [_vp, C.c_int32, _f32p, C.c_int32, _f32p, C.c_int32]),
    "t5h_set_profiling": (C.c_int, [_vp, C.c_int32]),
    "t5h_kernel_stats": (C.c_int, [_vp, C.POINTER(T5HKernelStat), C.c_int32]),
    "t5h_replay_kernel": (C.c_int, [_vp, C.c_int32, C.c_int32, C.POINTER(C.c_double)]),
}


class T5HError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"t5hip error {code}: {msg}")
        self.code = code


def load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                          "(make -C witchcraft_amd/csrc)")
    # torch ships its own libamdhip64.so.7 under the same soname as /opt/rocm's, and a process
    # holds one of them: whichever loads first serves both.  torch's CUDA init fails on a
    # runtime other than its own ("No HIP GPUs are available"), so when torch is installed
    # its copy is loaded first and this library binds to it.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = load()


def check(rc: int) -> None:
    if rc != T5H_OK:
        raise T5HError(rc, lib.t5h_last_error().decode(errors="replace"))
