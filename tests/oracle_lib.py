"""ctypes binding of the CPU oracle (oracle/ttlab_oracle.c).

Test infrastructure: the oracle is the checker the HIP path is compared against.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "build", "libttlab_oracle.so")

BODY_DEFAULT, BODY_V4, BODY_V4_SIMD = 0, 1, 2

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_szp = np.ctypeslib.ndpointer(dtype=np.uintp, flags="C_CONTIGUOUS")
_sz = C.c_size_t
_u64 = C.c_uint64


class MoeLayer(C.Structure):
    _fields_ = [
        ("hidden", C.c_size_t),
        ("expert_hidden", C.c_size_t),
        ("experts", C.c_size_t),
        ("used", C.c_size_t),
        ("router_weight", C.c_void_p),
        ("router_bias", C.c_void_p),
        ("gate_weight", C.c_void_p),
        ("gate_bias", C.c_void_p),
        ("up_weight", C.c_void_p),
        ("up_bias", C.c_void_p),
        ("down_weight", C.c_void_p),
        ("down_bias", C.c_void_p),
    ]


class OrcLayer(C.Structure):
    _fields_ = [
        ("attention_norm", C.c_void_p),
        ("post_attention_norm", C.c_void_p),
        ("query_weight", C.c_void_p),
        ("query_bias", C.c_void_p),
        ("key_weight", C.c_void_p),
        ("key_bias", C.c_void_p),
        ("value_weight", C.c_void_p),
        ("value_bias", C.c_void_p),
        ("output_weight", C.c_void_p),
        ("output_bias", C.c_void_p),
        ("sinks", C.c_void_p),
        ("moe", MoeLayer),
    ]


def _load():
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)
    lib = C.CDLL(ORACLE_SO)
    sig = {
        "orc_has_avx512": (C.c_int, []),
        "orc_mxfp4_scale": (C.c_float, [C.c_uint8]),
        "orc_mxfp4_int": (C.c_int, [C.c_uint8]),
        "orc_fp16_to_fp32": (C.c_float, [C.c_uint16]),
        "orc_fp32_to_bf16": (C.c_uint16, [C.c_float]),
        "orc_bf16_to_fp32": (C.c_float, [C.c_uint16]),
        "orc_mxfp4_dequant_blocks": (None, [_u8p, _sz, _f32p]),
        "orc_tensor_row_bytes": (C.c_int64, [C.c_uint32, C.c_uint64]),
        "orc_matvec_add_mxfp4": (None, [_u8p, _f32p, _sz, _sz, _f32p, _f32p, _sz, C.c_int]),
        "orc_transpose_selected": (None, [_sz, _f32p, _szp, _sz, _f32p]),
        "orc_matmul_add_mxfp4_selected_transposed": (
            None, [_u8p, _f32p, _sz, _sz, _f32p, _szp, _sz, _f32p, _f32p, _sz, C.c_int]),
        "orc_matvec_add_f32": (None, [_f32p, _f32p, _sz, _sz, _f32p, _f32p]),
        "orc_matmul_add_f32": (None, [_f32p, _f32p, _sz, _sz, _f32p, _sz, _f32p, _f32p, _f32p]),
        "orc_router_topk": (None, [_f32p, _sz, _sz, _i64p, _f32p]),
        "orc_swiglu": (None, [_f32p, _f32p, _sz, _f32p]),
        "orc_moe": (None, [C.POINTER(MoeLayer), _f32p, _f32p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]),
        "orc_moe_batch": (None, [C.POINTER(MoeLayer), _f32p, _sz, _f32p, C.c_int]),
        "orc_moe_batch_experts": (None, [C.POINTER(MoeLayer), _f32p, _sz, _i64p, _f32p, _f32p, C.c_int]),
        "orc_rope_frequencies": (None, [_f32p]),
        "orc_apply_rope": (None, [_f32p, _sz, _sz, _f32p]),
        "orc_attention": (None, [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _f32p, _f32p]),
        "orc_rms_norm": (None, [_f32p, _f32p, _sz, C.c_float, _f32p]),
        "orc_load_token_embedding_q8_0": (None, [_u8p, _sz, _sz, _f32p]),
        "orc_matvec_q8_0": (None, [_u8p, _sz, _sz, _f32p, _f32p]),
        "orc_matvec_add_q8_0": (None, [_u8p, _f32p, _sz, _sz, _f32p, _f32p]),
        "orc_matmul_add_q8_0": (None, [_u8p, _f32p, _sz, _sz, _f32p, _sz, _f32p, _f32p, _f32p]),
        "orc_matvec_bf16": (None, [_u16p, _sz, _sz, _f32p, _f32p]),
        "orc_greedy": (C.c_int32, [_f32p, _sz]),
        "orc_layer_prefill": (None, [C.POINTER(OrcLayer), _sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p, C.c_int, _f32p,
                                     C.c_void_p]),
        "orc_layer_forward": (None, [C.POINTER(OrcLayer), _sz, _sz, _f32p, _f32p, _f32p, _f32p, C.c_int, _f32p,
                                     _f32p, _f32p, _f32p, _f32p, _i64p, _f32p]),
        "orc_hash": (C.c_uint64, [_u64, _u64, _u64]),
        "orc_synth_normal": (None, [_u64, _u64, _sz, _sz, C.c_float, C.c_float, _f32p]),
        "orc_synth_normal_bf16": (None, [_u64, _u64, _sz, _sz, C.c_float, _f32p]),
        "orc_synth_mxfp4": (None, [_u64, _u64, _sz, _sz, C.c_uint32, C.c_uint32, _u8p]),
        "orc_synth_q8_0": (None, [_u64, _u64, _sz, _sz, _u8p]),
        "orc_synth_bf16": (None, [_u64, _u64, _sz, _sz, _u16p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def has_avx512():
    return bool(lib.orc_has_avx512())


# ---- convenience wrappers -------------------------------------------------

def mxfp4_matvec(matrix, bias, rows, cols, x, expert=0, body=BODY_DEFAULT):
    y = np.empty(rows, np.float32)
    lib.orc_matvec_add_mxfp4(matrix, bias, rows, cols, np.ascontiguousarray(x, np.float32), y, expert, body)
    return y


def synth_mxfp4(seed, stream, nblocks, emin=119, emax=125, block_offset=0):
    out = np.empty(nblocks * 17, np.uint8)
    lib.orc_synth_mxfp4(seed, stream, block_offset, nblocks, emin, emax, out)
    return out


def synth_normal(seed, stream, n, sigma=1.0, mean=0.0, offset=0):
    out = np.empty(n, np.float32)
    lib.orc_synth_normal(seed, stream, offset, n, mean, sigma, out)
    return out


def synth_normal_bf16(seed, stream, n, sigma, offset=0):
    out = np.empty(n, np.float32)
    lib.orc_synth_normal_bf16(seed, stream, offset, n, sigma, out)
    return out


def synth_q8_0(seed, stream, nblocks, block_offset=0):
    out = np.empty(nblocks * 34, np.uint8)
    lib.orc_synth_q8_0(seed, stream, block_offset, nblocks, out)
    return out


def synth_bf16(seed, stream, n, offset=0):
    out = np.empty(n, np.uint16)
    lib.orc_synth_bf16(seed, stream, offset, n, out)
    return out


def dequant_mxfp4(blocks):
    n = blocks.size // 17
    out = np.empty(n * 32, np.float32)
    lib.orc_mxfp4_dequant_blocks(np.ascontiguousarray(blocks), n, out)
    return out


def router_topk(logits, k=4):
    logits = np.ascontiguousarray(logits, np.float32)
    idx = np.empty(k, np.int64)
    w = np.empty(k, np.float32)
    lib.orc_router_topk(logits, logits.size, k, idx, w)
    return idx, w


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
