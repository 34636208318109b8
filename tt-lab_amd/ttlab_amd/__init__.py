"""ctypes binding of the gfx950 backend's C ABI (include/ttlab_hip.h).

The product is the shared library build/libttlab_hip.so; this module only loads
it and wraps its entry points for Python callers (tests, bench.py).  There is no
fallback: if the library is missing or the GPU is absent, calls raise.
"""
import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "build", "libttlab_hip.so")
HEADER_PATH = os.path.join(REPO_DIR, "include", "ttlab_hip.h")

TTL_OK = 0
TTL_DTYPE_F32 = 0
TTL_DTYPE_BF16 = 1
TTL_DTYPE_F32_AS_MXFP8 = 2
TTL_DTYPE_BF16_AS_MXFP8 = 3
TTL_PREFILL_PLAN, TTL_PREFILL_GATHER, TTL_PREFILL_GATEUP, TTL_PREFILL_DOWN, TTL_PREFILL_COMBINE = 1, 2, 4, 8, 16
TTL_PREFILL_ALL = 31


class TtlError(RuntimeError):
    pass


class MoeLayerDesc(C.Structure):
    """Mirror of ttl_moe_layer."""
    _fields_ = [
        ("hidden", C.c_uint32),
        ("expert_hidden", C.c_uint32),
        ("experts", C.c_uint32),
        ("used", C.c_uint32),
        ("router_weight", C.c_void_p),
        ("router_bias", C.c_void_p),
        ("gate", C.c_void_p),
        ("gate_bias", C.c_void_p),
        ("up", C.c_void_p),
        ("up_bias", C.c_void_p),
        ("down", C.c_void_p),
        ("down_bias", C.c_void_p),
        ("input_norm", C.c_void_p),
        ("input_norm_epsilon", C.c_float),
    ]


class StageInput(C.Structure):
    """Mirror of ttl_stage_input."""
    _fields_ = [
        ("base", C.c_void_p),
        ("add", C.c_void_p),
        ("add_weights", C.c_void_p),
        ("add_count", C.c_uint32),
        ("norm_weight", C.c_void_p),
        ("epsilon", C.c_float),
        ("sum_out", C.c_void_p),
    ]


def stage_input(base, add=None, add_weights=None, add_count=0, norm=None, eps=1e-5, sum_out=None):
    s = StageInput()
    s.base = base.ptr
    s.add = add.ptr if add else None
    s.add_weights = add_weights.ptr if add_weights else None
    s.add_count = add_count
    s.norm_weight = norm.ptr if norm else None
    s.epsilon = eps
    s.sum_out = sum_out.ptr if sum_out else None
    return s


_lib = None
_model_lib = None
MODEL_LIB_PATH = os.path.join(PKG_DIR, "build", "libttlab_model.so")


def load_model_library():
    """Loads build/libttlab_model.so (the C++ HipGptOssModel behind include/ttlab_model.h)."""
    global _model_lib
    if _model_lib is not None:
        return _model_lib
    load_library()
    if not os.path.exists(MODEL_LIB_PATH):
        raise TtlError(f"{MODEL_LIB_PATH} is missing: run __graft_entry__.build()")
    lib = C.CDLL(MODEL_LIB_PATH)
    vp, u32, u64, i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int
    sigs = {
        "ttlm_create_synthetic": (i32, [i32, u32, u32, u32, u32, C.c_uint64, C.POINTER(vp)]),
        "ttlm_destroy": (None, [vp]),
        "ttlm_last_error": (C.c_char_p, []),
        "ttlm_forward": (i32, [vp, C.c_int32, u32, vp]),
        "ttlm_prefill": (i32, [vp, vp, u32, vp]),
        "ttlm_generate": (i32, [vp, C.c_int32, u32, u32, vp]),
        "ttlm_time_decode": (i32, [vp, C.c_int32, u32, u32, u32, C.POINTER(C.c_double)]),
        "ttlm_time_expert_kernel": (i32, [vp, u32, C.POINTER(C.c_double)]),
        "ttlm_set_graph_replay": (i32, [vp, i32]),
        "ttlm_time_kernel": (i32, [vp, u32, u32, u32, C.POINTER(C.c_double), C.POINTER(u32)]),
        "ttlm_layer_state": (i32, [vp, u32, vp, vp, vp, vp]),
        "ttlm_final_state": (i32, [vp, vp]),
        "ttlm_kv_cache": (i32, [vp, u32, u32, vp, vp]),
        "ttlm_fill_kv_synthetic": (i32, [vp, u32, u64]),
        "ttlm_device_bytes": (C.c_size_t, [vp]),
        "ttlm_step_bytes": (C.c_double, [vp, u32]),
        "ttlm_prefill_state": (i32, [vp, u32, u32, vp]),
        "ttlm_prefill_batch": (u32, [vp]),
        "ttlm_gguf_inspect": (i32, [C.c_char_p, i32, C.POINTER(GgufInfo)]),
        "ttlm_create_from_gguf": (i32, [C.c_char_p, i32, u32, i32, C.POINTER(vp)]),
        "ttlm_tokenizer_open": (i32, [C.c_char_p, C.POINTER(vp)]),
        "ttlm_tokenizer_free": (None, [vp]),
        "ttlm_tokenizer_encode": (i32, [vp, C.c_char_p, C.c_size_t, vp, C.c_size_t, C.POINTER(C.c_size_t)]),
        "ttlm_tokenizer_decode": (i32, [vp, C.c_int32, i32, vp, C.c_size_t, C.POINTER(C.c_size_t)]),
        "ttlm_tokenizer_vocabulary": (C.c_size_t, [vp]),
        "ttlm_pretokenize": (i32, [C.c_char_p, C.c_size_t, vp, C.c_size_t, C.POINTER(C.c_size_t)]),
        "ttlm_harmony_prompt": (C.c_size_t, [C.c_char_p, C.c_size_t, vp, C.c_size_t]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _model_lib = lib
    return lib


def _mcheck(rc, what):
    if rc != 0:
        msg = load_model_library().ttlm_last_error()
        raise TtlError(f"{what} failed: {msg.decode() if msg else ''}")


class Tokenizer:
    """ttlab::Tokenizer (include/ttlab_model.h, ttlm_tokenizer_*): the gpt-oss BPE of a
    GGUF file's tokenizer.ggml.* metadata, as the reference's Tokenizer."""

    def __init__(self, path):
        self.lib = load_model_library()
        h = C.c_void_p()
        _mcheck(self.lib.ttlm_tokenizer_open(os.fsencode(path), C.byref(h)), "ttlm_tokenizer_open")
        self.handle = h

    def encode(self, text):
        data = text.encode() if isinstance(text, str) else bytes(text)
        count = C.c_size_t()
        cap = 4 * len(data) + 16
        out = (C.c_int32 * cap)()
        _mcheck(self.lib.ttlm_tokenizer_encode(self.handle, data, len(data), out, cap, C.byref(count)),
                "ttlm_tokenizer_encode")
        assert count.value <= cap
        return list(out[:count.value])

    def decode(self, token, render_special=True, capacity=1024):
        """The token's bytes (bytes object); raises TtlError as the reference throws."""
        buf = C.create_string_buffer(max(capacity, 1))
        n = C.c_size_t()
        _mcheck(self.lib.ttlm_tokenizer_decode(self.handle, token, 1 if render_special else 0, buf, capacity,
                                               C.byref(n)), "ttlm_tokenizer_decode")
        return buf.raw[:n.value]

    def vocabulary(self):
        return self.lib.ttlm_tokenizer_vocabulary(self.handle)

    def close(self):
        if self.handle:
            self.lib.ttlm_tokenizer_free(self.handle)
            self.handle = None


def pretokenize(text):
    """The gpt-4o pre-tokenizer's pieces (bytes) under the process's LC_CTYPE."""
    lib = load_model_library()
    data = text.encode() if isinstance(text, str) else bytes(text)
    cap = len(data) + 1
    ends = (C.c_size_t * cap)()
    count = C.c_size_t()
    _mcheck(lib.ttlm_pretokenize(data, len(data), ends, cap, C.byref(count)), "ttlm_pretokenize")
    pieces, start = [], 0
    for k in range(count.value):
        pieces.append(data[start:ends[k]])
        start = ends[k]
    return pieces


def harmony_prompt(user):
    lib = load_model_library()
    data = user.encode() if isinstance(user, str) else bytes(user)
    n = lib.ttlm_harmony_prompt(data, len(data), None, 0)
    buf = C.create_string_buffer(n + 1)
    lib.ttlm_harmony_prompt(data, len(data), buf, n)
    return buf.raw[:n]


class GgufInfo(C.Structure):
    """Mirror of ttlm_gguf_info."""
    _fields_ = [("layers", C.c_uint32), ("experts", C.c_uint32), ("vocab", C.c_uint32), ("output_type", C.c_uint32),
                ("tensors", C.c_uint32)]


def gguf_inspect(path, strict=True):
    """The reference's checks of a gpt-oss GGUF file (no device needed); raises TtlError."""
    lib = load_model_library()
    info = GgufInfo()
    _mcheck(lib.ttlm_gguf_inspect(os.fsencode(path), 1 if strict else 0, C.byref(info)), "ttlm_gguf_inspect")
    return {k: getattr(info, k) for k, _ in GgufInfo._fields_}


class Model:
    """ttlab::HipGptOssModel with synthetic weights (benchmark configurations 3/4), or
    with a GGUF file's weights (Model.from_gguf)."""

    def __init__(self, layers=24, experts=32, vocab=201088, capacity=2112, seed=0x77000003, device=0, _handle=None):
        self.lib = load_model_library()
        if _handle is None:
            p = C.c_void_p()
            _mcheck(self.lib.ttlm_create_synthetic(device, layers, experts, vocab, capacity, seed, C.byref(p)),
                    "ttlm_create_synthetic")
            _handle = p.value
        self.h = _handle
        self.layers, self.experts, self.vocab, self.capacity, self.seed = layers, experts, vocab, capacity, seed

    @classmethod
    def from_gguf(cls, path, capacity, strict=True, device=0):
        lib = load_model_library()
        info = gguf_inspect(path, strict)
        p = C.c_void_p()
        _mcheck(lib.ttlm_create_from_gguf(os.fsencode(path), device, capacity, 1 if strict else 0, C.byref(p)),
                "ttlm_create_from_gguf")
        return cls(info["layers"], info["experts"], info["vocab"], capacity, 0, device, _handle=p.value)

    def close(self):
        if self.h:
            self.lib.ttlm_destroy(self.h)
            self.h = None

    def forward(self, token, position):
        out = np.empty(self.vocab, np.float32)
        _mcheck(self.lib.ttlm_forward(self.h, token, position, out.ctypes.data), "ttlm_forward")
        return out

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.vocab, np.float32)
        _mcheck(self.lib.ttlm_prefill(self.h, t.ctypes.data, t.size, out.ctypes.data), "ttlm_prefill")
        return out

    def prefill_state(self, layer, count):
        out = np.empty(count * 2880, np.float32)
        _mcheck(self.lib.ttlm_prefill_state(self.h, layer, count, out.ctypes.data), "ttlm_prefill_state")
        return out.reshape(count, 2880)

    @property
    def prefill_batch(self):
        return int(self.lib.ttlm_prefill_batch(self.h))

    def fill_kv_synthetic(self, positions, seed=0x78000300):
        """KV caches of every layer filled with N(0, 1) values for positions [0, positions)."""
        _mcheck(self.lib.ttlm_fill_kv_synthetic(self.h, positions, seed), "ttlm_fill_kv_synthetic")

    def generate(self, token, position, steps):
        out = np.empty(steps, np.int32)
        _mcheck(self.lib.ttlm_generate(self.h, token, position, steps, out.ctypes.data), "ttlm_generate")
        return out

    def time_decode(self, token, position, warmup, steps):
        ms = C.c_double()
        _mcheck(self.lib.ttlm_time_decode(self.h, token, position, warmup, steps, C.byref(ms)), "ttlm_time_decode")
        return ms.value

    def time_expert_kernel(self, reps):
        us = C.c_double()
        _mcheck(self.lib.ttlm_time_expert_kernel(self.h, reps, C.byref(us)), "ttlm_time_expert_kernel")
        return us.value

    def set_graph_replay(self, enabled):
        _mcheck(self.lib.ttlm_set_graph_replay(self.h, 1 if enabled else 0), "ttlm_set_graph_replay")

    KERNELS = ("qkv", "attention_window", "attention_full", "output", "router_rows", "gateup_routed",
               "gateup_given", "down", "logits", "gateup_down")

    def time_kernel(self, kind, position, reps):
        """Microseconds per launch of one kind of the step's kernels (KERNELS names them), and
        the launches per step."""
        us, n = C.c_double(), C.c_uint32()
        _mcheck(self.lib.ttlm_time_kernel(self.h, self.KERNELS.index(kind), position, reps, C.byref(us), C.byref(n)),
                "ttlm_time_kernel")
        return us.value, n.value

    def layer_state(self, layer):
        x = np.empty(2880, np.float32)
        r = np.empty(2880, np.float32)
        idx = np.empty(4, np.int32)
        w = np.empty(4, np.float32)
        _mcheck(self.lib.ttlm_layer_state(self.h, layer, x.ctypes.data, r.ctypes.data, idx.ctypes.data,
                                          w.ctypes.data), "ttlm_layer_state")
        return x, r, idx, w

    def final_state(self):
        x = np.empty(2880, np.float32)
        _mcheck(self.lib.ttlm_final_state(self.h, x.ctypes.data), "ttlm_final_state")
        return x

    def kv_cache(self, layer, positions):
        k = np.empty(positions * 512, np.float32)
        v = np.empty(positions * 512, np.float32)
        _mcheck(self.lib.ttlm_kv_cache(self.h, layer, positions, k.ctypes.data, v.ctypes.data), "ttlm_kv_cache")
        return k, v

    @property
    def device_bytes(self):
        return self.lib.ttlm_device_bytes(self.h)

    def step_bytes(self, position):
        return self.lib.ttlm_step_bytes(self.h, position)


def load_library():
    """Loads build/libttlab_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise TtlError(f"{LIB_PATH} is missing: run __graft_entry__.build() (make -C tt-lab_amd)")
    lib = C.CDLL(LIB_PATH)
    vp, u32, u64, sz, f32, i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_size_t, C.c_float, C.c_int
    sigs = {
        "ttl_create": (i32, [i32, C.POINTER(vp)]),
        "ttl_destroy": (None, [vp]),
        "ttl_last_error": (C.c_char_p, []),
        "ttl_sync": (i32, [vp]),
        "ttl_device_info": (i32, [vp, C.c_char_p, sz, C.POINTER(i32), C.POINTER(C.c_double)]),
        "ttl_malloc": (i32, [vp, sz, C.POINTER(vp)]),
        "ttl_free": (i32, [vp, vp]),
        "ttl_memcpy_h2d": (i32, [vp, vp, vp, sz]),
        "ttl_memcpy_d2h": (i32, [vp, vp, vp, sz]),
        "ttl_memcpy_d2d": (i32, [vp, vp, vp, sz]),
        "ttl_fill_bytes": (i32, [vp, vp, C.c_uint8, sz]),
        "ttl_timer_start": (i32, [vp]),
        "ttl_timer_stop": (i32, [vp, C.POINTER(f32)]),
        "ttl_synth_normal": (i32, [vp, u64, u64, sz, sz, f32, f32, vp]),
        "ttl_synth_normal_bf16": (i32, [vp, u64, u64, sz, sz, f32, vp]),
        "ttl_synth_mxfp4_gguf": (i32, [vp, u64, u64, sz, sz, u32, u32, vp]),
        "ttl_mxfp4_upload": (i32, [vp, vp, u32, u32, u32, C.POINTER(vp)]),
        "ttl_mxfp4_upload_dev": (i32, [vp, vp, u32, u32, u32, C.POINTER(vp)]),
        "ttl_mxfp4_synthetic": (i32, [vp, u32, u32, u32, u64, u64, u32, u32, C.POINTER(vp)]),
        "ttl_mxfp4_download": (i32, [vp, vp, vp]),
        "ttl_mxfp4_free": (None, [vp, vp]),
        "ttl_mxfp4_shape": (i32, [vp, C.POINTER(u32), C.POINTER(u32), C.POINTER(u32)]),
        "ttl_mxfp4_bytes": (sz, [vp]),
        "ttl_mxfp4_edge_scales": (i32, [vp]),
        "ttl_mxfp4_f16_exact": (i32, [vp]),
        "ttl_mxfp4_dequantize": (i32, [vp, vp, u32, i32, vp]),
        "ttl_matvec_mxfp4": (i32, [vp, vp, vp, vp, vp, u32]),
        "ttl_matvec_mxfp4_experts": (i32, [vp, vp, vp, vp, u32, vp, u32, vp]),
        "ttl_router_topk": (i32, [vp, vp, vp, u32, u32, vp, u32, u32, vp, vp, vp]),
        "ttl_router_exact_count": (i32, [vp, C.POINTER(u64)]),
        "ttl_moe_decode": (i32, [vp, C.POINTER(MoeLayerDesc), vp, vp, vp, vp]),
        "ttl_moe_gateup_swiglu": (i32, [vp, C.POINTER(MoeLayerDesc), vp, vp, vp]),
        "ttl_moe_down": (i32, [vp, C.POINTER(MoeLayerDesc), vp, vp, vp]),
        "ttl_moe_combine": (i32, [vp, vp, vp, u32, u32, vp]),
        "ttl_moe_down_combine": (i32, [vp, vp, vp, vp, vp, vp, vp, vp]),
        "ttl_moe_route_gateup": (i32, [vp, C.POINTER(MoeLayerDesc), vp, vp, vp, vp]),
        "ttl_moe_route_gateup_down": (i32, [vp, C.POINTER(MoeLayerDesc), vp, vp, vp, vp, vp, u32]),
        "ttl_moe_gateup_down_fused": (i32, [vp, C.POINTER(MoeLayerDesc), C.POINTER(C.c_int)]),
        "ttl_moe_handoff_give_ups": (i32, [vp, C.POINTER(C.c_uint64)]),
        "ttl_synth_bf16": (i32, [vp, u64, u64, sz, sz, vp]),
        "ttl_q8_upload": (i32, [vp, vp, u32, u32, vp, u32, C.POINTER(vp)]),
        "ttl_q8_upload_dev": (i32, [vp, vp, u32, u32, vp, C.POINTER(vp)]),
        "ttl_q8_download": (i32, [vp, vp, vp]),
        "ttl_q8_free": (None, [vp, vp]),
        "ttl_q8_bytes": (sz, [vp]),
        "ttl_synth_q8_0_gguf": (i32, [vp, u64, u64, sz, sz, vp]),
        "ttl_matvec_q8_0": (i32, [vp, vp, vp, C.POINTER(StageInput), vp, vp]),
        "ttl_qkv_row_source": (i32, [vp]),
        "ttl_attn_qkv": (i32, [vp, vp, vp, C.POINTER(StageInput), vp, vp, u32, vp, vp, vp]),
        "ttl_attention_workspace_bytes": (sz, [u32]),
        "ttl_attention_decode": (i32, [vp, vp, vp, vp, vp, vp, u32, u32, vp, vp]),
        "ttl_attention_decode_noalloc": (i32, [vp, vp, vp, vp, vp, vp, u32, u32, vp]),
        "ttl_attention_prefill": (i32, [vp, vp, vp, vp, vp, u32, u32, u32, u32, vp]),
        "ttl_embedding_q8_0": (i32, [vp, vp, u32, vp, vp]),
        "ttl_logits_workspace_bytes": (sz, [u32]),
        "ttl_logits_bf16": (i32, [vp, vp, u32, C.POINTER(StageInput), vp, vp]),
        "ttl_argmax": (i32, [vp, u32, vp, vp, vp, vp, u32]),
        "ttl_matmul_mxfp4_selected_workspace_bytes": (sz, [u32]),
        "ttl_matmul_mxfp4_selected": (i32, [vp, vp, vp, vp, u32, u32, vp, u32, vp, u32, vp, sz]),
        "ttl_matmul_mxfp4_selected_mxfp8_workspace_bytes": (sz, [u32]),
        "ttl_matmul_mxfp4_selected_mxfp8": (i32, [vp, vp, vp, vp, u32, u32, vp, u32, vp, u32, vp, sz]),
        "ttl_mxfp8_dequantize": (i32, [vp, vp, i32, u32, vp]),
        "ttl_moe_prefill_workspace_bytes": (sz, [u32, u32, u32, i32]),
        "ttl_moe_prefill_experts": (i32, [vp, C.POINTER(MoeLayerDesc), vp, i32, u32, vp, vp, vp, vp, sz]),
        "ttl_moe_prefill_stages": (i32, [vp, C.POINTER(MoeLayerDesc), vp, i32, u32, vp, vp, vp, vp, sz, u32]),
        "ttl_moe_prefill_intermediates": (i32, [vp, C.POINTER(MoeLayerDesc), i32, u32, vp, sz, vp, vp, vp]),
        "ttl_moe_prefill_batch_workspace_bytes": (sz, [u32, u32, u32]),
        "ttl_moe_prefill": (i32, [vp, C.POINTER(MoeLayerDesc), vp, u32, vp, vp, vp, vp, sz]),
        "ttl_moe_prefill_fused": (i32, [vp, C.POINTER(MoeLayerDesc), vp, vp, vp, u32, vp, vp, vp, vp, sz]),
        "ttl_rms_norm_rows": (i32, [vp, vp, u32, vp, f32, vp]),
        "ttl_rms_norm_rows_shifts": (i32, [vp, vp, u32, vp, f32, vp, vp]),
        "ttl_logits_q8_0": (i32, [vp, vp, u32, C.POINTER(StageInput), vp, vp]),
        "ttl_stream_read": (i32, [vp, vp, sz, vp]),
        "ttl_measure_handoff": (i32, [vp, i32, u32, C.POINTER(f32), C.POINTER(u32)]),
        "ttl_measure_boundary": (i32, [vp, u32, u32, u32, C.POINTER(f32), C.POINTER(u32)]),
        "ttl_stream_read_plain": (i32, [vp, vp, sz, vp]),
        "ttl_matmul_q8_0_workspace_bytes": (sz, [u32, u32]),
        "ttl_matmul_q8_0": (i32, [vp, vp, vp, vp, u32, vp, vp, vp, sz]),
        "ttl_matmul_q8_0_shifted": (i32, [vp, vp, vp, vp, vp, u32, vp, vp, vp, sz]),
        "ttl_capture_begin": (i32, [vp]),
        "ttl_capture_end": (i32, [vp, C.POINTER(vp)]),
        "ttl_graph_launch": (i32, [vp, vp]),
        "ttl_graph_free": (None, [vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def balanced_routing(count, experts, used, seed):
    """Synthetic routing of benchmark config 2: every expert is chosen equally often,
    each token has `used` distinct experts (rank order shuffled), and the weights are
    the softmax of N(0,1) logits.  Returns int32 [count][used], f32 [count][used]."""
    if (count * used) % experts or experts % used:
        raise ValueError("balanced routing needs experts | count*used and used | experts")
    rng = np.random.RandomState(seed)
    step = experts // used
    base = np.arange(count) % experts
    idx = np.stack([(base + step * r) % experts for r in range(used)], axis=1)
    labels = rng.permutation(experts)
    idx = labels[idx][rng.permutation(count)]
    for p in range(count):
        idx[p] = idx[p][rng.permutation(used)]
    logits = rng.randn(count, used)
    w = np.exp(logits - logits.max(1, keepdims=True))
    return idx.astype(np.int32), (w / w.sum(1, keepdims=True)).astype(np.float32)


def bf16_bits(values):
    """f32 -> bf16 bit patterns, round to nearest even (requant.cpp:311-316 for finite values)."""
    u = np.ascontiguousarray(values, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def header_symbols():
    """Names of the functions include/ttlab_hip.h declares."""
    import re
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ttl_[a-z0-9_]+)\s*\(", text)))


def _check(rc, what):
    if rc != TTL_OK:
        msg = load_library().ttl_last_error()
        raise TtlError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")


class Buffer:
    """Device allocation owned by a Device."""

    def __init__(self, dev, nbytes):
        self.dev = dev
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(dev.lib.ttl_malloc(dev.ctx, self.nbytes, C.byref(p)), "ttl_malloc")
        self.ptr = p.value

    def free(self):
        if self.ptr:
            self.dev.lib.ttl_free(self.dev.ctx, self.ptr)
            self.ptr = None

    def offset(self, nbytes):
        return C.c_void_p(self.ptr + int(nbytes))

    @property
    def p(self):
        return C.c_void_p(self.ptr)

    def upload(self, array):
        a = np.ascontiguousarray(array)
        assert a.nbytes <= self.nbytes
        _check(self.dev.lib.ttl_memcpy_h2d(self.dev.ctx, self.ptr, a.ctypes.data, a.nbytes), "ttl_memcpy_h2d")
        return self

    def download(self, dtype, count=None, offset_bytes=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset_bytes) // dtype.itemsize
        out = np.empty(count, dtype)
        _check(self.dev.lib.ttl_memcpy_d2h(self.dev.ctx, out.ctypes.data, self.ptr + offset_bytes, out.nbytes),
               "ttl_memcpy_d2h")
        return out


class Mxfp4:
    """Device MXFP4 tensor handle (ttl_mxfp4)."""

    def __init__(self, dev, handle):
        self.dev = dev
        self.handle = handle
        r, c, e = C.c_uint32(), C.c_uint32(), C.c_uint32()
        _check(dev.lib.ttl_mxfp4_shape(handle, C.byref(r), C.byref(c), C.byref(e)), "ttl_mxfp4_shape")
        self.rows, self.cols, self.experts = r.value, c.value, e.value

    @property
    def nbytes(self):
        return self.dev.lib.ttl_mxfp4_bytes(self.handle)

    @property
    def edge_scales(self):
        """True if some block has E8M0 scale 0 or 255 (the MFMA entry points refuse it)."""
        rc = self.dev.lib.ttl_mxfp4_edge_scales(self.handle)
        if rc < 0:
            _check(rc, "ttl_mxfp4_edge_scales")
        return bool(rc)

    @property
    def f16_exact(self):
        """True if every nonzero block's E8M0 scale is 114..140 (the f16 down GEMM's range)."""
        rc = self.dev.lib.ttl_mxfp4_f16_exact(self.handle)
        if rc < 0:
            _check(rc, "ttl_mxfp4_f16_exact")
        return bool(rc)

    def download_gguf(self):
        out = np.empty(self.rows * self.cols // 32 * 17 * self.experts, np.uint8)
        _check(self.dev.lib.ttl_mxfp4_download(self.dev.ctx, self.handle, out.ctypes.data), "ttl_mxfp4_download")
        return out

    def dequantize(self, expert, mode=0):
        buf = self.dev.alloc(self.rows * self.cols * 4)
        try:
            _check(self.dev.lib.ttl_mxfp4_dequantize(self.dev.ctx, self.handle, expert, mode, buf.ptr),
                   "ttl_mxfp4_dequantize")
            return buf.download(np.float32).reshape(self.rows, self.cols)
        finally:
            buf.free()

    def free(self):
        if self.handle:
            self.dev.lib.ttl_mxfp4_free(self.dev.ctx, self.handle)
            self.handle = None


class Q8:
    """Device Q8_0 tensor handle (ttl_q8)."""

    def __init__(self, dev, handle, rows, cols):
        self.dev, self.handle, self.rows, self.cols = dev, handle, rows, cols

    def download_gguf(self):
        out = np.empty(self.rows * self.cols // 32 * 34, np.uint8)
        _check(self.dev.lib.ttl_q8_download(self.dev.ctx, self.handle, out.ctypes.data), "ttl_q8_download")
        return out

    def free(self):
        if self.handle:
            self.dev.lib.ttl_q8_free(self.dev.ctx, self.handle)
            self.handle = None


class Graph:
    """Instantiated HIP graph (ttl_graph)."""

    def __init__(self, dev, handle):
        self.dev, self.handle = dev, handle

    def launch(self):
        _check(self.dev.lib.ttl_graph_launch(self.dev.ctx, self.handle), "ttl_graph_launch")

    def free(self):
        if self.handle:
            self.dev.lib.ttl_graph_free(self.handle)
            self.handle = None


class Device:
    """One ttl_ctx: a gfx950 device and its stream."""

    def __init__(self, ordinal=0):
        self.lib = load_library()
        p = C.c_void_p()
        _check(self.lib.ttl_create(ordinal, C.byref(p)), "ttl_create")
        self.ctx = p.value

    def close(self):
        if self.ctx:
            self.lib.ttl_destroy(self.ctx)
            self.ctx = None

    def info(self):
        name = C.create_string_buffer(128)
        cu = C.c_int()
        mem = C.c_double()
        _check(self.lib.ttl_device_info(self.ctx, name, 128, C.byref(cu), C.byref(mem)), "ttl_device_info")
        return {"name": name.value.decode(), "compute_units": cu.value, "hbm_bytes": mem.value}

    def sync(self):
        _check(self.lib.ttl_sync(self.ctx), "ttl_sync")

    def alloc(self, nbytes):
        return Buffer(self, nbytes)

    def upload(self, array):
        a = np.ascontiguousarray(array)
        return Buffer(self, max(a.nbytes, 1)).upload(a)

    def fill(self, buf, value, nbytes=None):
        _check(self.lib.ttl_fill_bytes(self.ctx, buf.ptr, value, buf.nbytes if nbytes is None else nbytes),
               "ttl_fill_bytes")

    def copy(self, dst, src, nbytes):
        """Device-to-device copy; dst/src are Buffers or device pointers (Buffer.offset)."""
        d = dst.ptr if isinstance(dst, Buffer) else dst
        s = src.ptr if isinstance(src, Buffer) else src
        _check(self.lib.ttl_memcpy_d2d(self.ctx, d, s, nbytes), "ttl_memcpy_d2d")

    def timer_start(self):
        _check(self.lib.ttl_timer_start(self.ctx), "ttl_timer_start")

    def timer_stop(self):
        ms = C.c_float()
        _check(self.lib.ttl_timer_stop(self.ctx, C.byref(ms)), "ttl_timer_stop")
        return ms.value

    def measure_handoff(self, mode, launches=50):
        """(microseconds per handoff, consumers that saw a wrong sum or gave up):
        mode 0 across a kernel boundary, mode 1 inside one kernel."""
        us, wrong = C.c_float(), C.c_uint32()
        _check(self.lib.ttl_measure_handoff(self.ctx, mode, launches, C.byref(us), C.byref(wrong)),
               "ttl_measure_handoff")
        return us.value, wrong.value

    def measure_boundary(self, launches=200, blocks=1, threads=64):
        """(microseconds per launch of a chain of dependent kernels, 1 if the chain's count
        came out wrong): the fixed cost of a kernel boundary in a replayed graph."""
        us, wrong = C.c_float(), C.c_uint32()
        _check(self.lib.ttl_measure_boundary(self.ctx, launches, blocks, threads, C.byref(us), C.byref(wrong)),
               "ttl_measure_boundary")
        return us.value, wrong.value

    def time_stream_read(self, buffers, nbytes, nontemporal=True, reps=20):
        """Microseconds per launch of a plain read of nbytes (non-temporal or ordinary loads),
        over the given buffers in turn, captured as one graph and replayed."""
        sink = self.alloc(256)
        fn = self.lib.ttl_stream_read if nontemporal else self.lib.ttl_stream_read_plain

        def launches():
            for b in buffers:
                _check(fn(self.ctx, b.ptr, nbytes, sink.ptr), "stream read")

        g = self.capture(launches)
        for _ in range(3):
            g.launch()
        self.sync()
        self.timer_start()
        for _ in range(reps):
            g.launch()
        us = 1e3 * self.timer_stop() / (reps * len(buffers))
        g.free()
        sink.free()
        return us

    # ---- synthetic inputs ----
    def synth_normal(self, buf, seed, stream, n, sigma=1.0, mean=0.0, offset=0):
        _check(self.lib.ttl_synth_normal(self.ctx, seed, stream, offset, n, mean, sigma, buf.ptr), "ttl_synth_normal")

    def synth_normal_bf16(self, buf, seed, stream, n, sigma, offset=0):
        _check(self.lib.ttl_synth_normal_bf16(self.ctx, seed, stream, offset, n, sigma, buf.ptr),
               "ttl_synth_normal_bf16")

    def synth_mxfp4_gguf(self, buf, seed, stream, nblocks, emin=119, emax=125, block_offset=0):
        _check(self.lib.ttl_synth_mxfp4_gguf(self.ctx, seed, stream, block_offset, nblocks, emin, emax, buf.ptr),
               "ttl_synth_mxfp4_gguf")

    # ---- MXFP4 ----
    def mxfp4_upload(self, gguf_bytes, rows, cols, experts):
        a = np.ascontiguousarray(gguf_bytes, np.uint8)
        h = C.c_void_p()
        _check(self.lib.ttl_mxfp4_upload(self.ctx, a.ctypes.data, rows, cols, experts, C.byref(h)), "ttl_mxfp4_upload")
        return Mxfp4(self, h.value)

    def mxfp4_synthetic(self, rows, cols, experts, seed, stream, emin=119, emax=125):
        h = C.c_void_p()
        _check(self.lib.ttl_mxfp4_synthetic(self.ctx, rows, cols, experts, seed, stream, emin, emax, C.byref(h)),
               "ttl_mxfp4_synthetic")
        return Mxfp4(self, h.value)

    def matvec_mxfp4(self, w, bias, x, y, expert):
        _check(self.lib.ttl_matvec_mxfp4(self.ctx, w.handle, bias.ptr if bias else None, x.ptr, y.ptr, expert),
               "ttl_matvec_mxfp4")

    def router_topk(self, weight, bias, experts, x, k, logits, indices, weights, force_exact=False):
        _check(self.lib.ttl_router_topk(self.ctx, weight.ptr, bias.ptr, experts, 2880, x.ptr, k,
                                        1 if force_exact else 0, logits.ptr, indices.ptr, weights.ptr),
               "ttl_router_topk")

    def router_exact_count(self):
        c = C.c_uint64()
        _check(self.lib.ttl_router_exact_count(self.ctx, C.byref(c)), "ttl_router_exact_count")
        return c.value

    def moe_decode(self, layer, x, out, indices=None, weights=None):
        _check(self.lib.ttl_moe_decode(self.ctx, C.byref(layer), x.ptr, out.ptr, indices.ptr if indices else None,
                                       weights.ptr if weights else None), "ttl_moe_decode")

    def moe_gateup_swiglu(self, layer, x, indices, hidden):
        _check(self.lib.ttl_moe_gateup_swiglu(self.ctx, C.byref(layer), x.ptr, indices.ptr, hidden.ptr),
               "ttl_moe_gateup_swiglu")

    def moe_route_gateup(self, layer, x, hidden, indices, weights):
        _check(self.lib.ttl_moe_route_gateup(self.ctx, C.byref(layer), x.ptr, hidden.ptr, indices.ptr, weights.ptr),
               "ttl_moe_route_gateup")

    def moe_route_gateup_down(self, layer, x, hidden, indices, weights, down, stages=5):
        """Router rows (stage 1), then gate/up + down in one launch (stage 4)."""
        _check(self.lib.ttl_moe_route_gateup_down(self.ctx, C.byref(layer), x.ptr, hidden.ptr, indices.ptr,
                                                  weights.ptr, down.ptr, stages), "ttl_moe_route_gateup_down")

    def moe_gateup_down_fused(self, layer):
        f = C.c_int()
        _check(self.lib.ttl_moe_gateup_down_fused(self.ctx, C.byref(layer), C.byref(f)), "ttl_moe_gateup_down_fused")
        return bool(f.value)

    def handoff_give_ups(self):
        c = C.c_uint64()
        _check(self.lib.ttl_moe_handoff_give_ups(self.ctx, C.byref(c)), "ttl_moe_handoff_give_ups")
        return c.value

    def moe_down(self, layer, hidden, indices, down):
        _check(self.lib.ttl_moe_down(self.ctx, C.byref(layer), hidden.ptr, indices.ptr, down.ptr), "ttl_moe_down")

    def moe_down_combine(self, layer, hidden, indices, weights, residual, out, down=None):
        _check(self.lib.ttl_moe_down_combine(self.ctx, C.byref(layer), hidden.p, indices.p, weights.p,
                                             residual.p if residual is not None else None, out.p,
                                             down.p if down is not None else None), "ttl_moe_down_combine")

    def moe_combine(self, down, weights, k, n, out):
        _check(self.lib.ttl_moe_combine(self.ctx, down.ptr, weights.ptr, k, n, out.ptr), "ttl_moe_combine")

    # ---- Q8_0 / attention / logits ----
    def q8_upload(self, gguf_bytes, rows, cols, row_source=None, source_rows=None):
        a = np.ascontiguousarray(gguf_bytes, np.uint8)
        rs = None if row_source is None else np.ascontiguousarray(row_source, np.int32)
        h = C.c_void_p()
        _check(self.lib.ttl_q8_upload(self.ctx, a.ctypes.data, rows, cols, None if rs is None else rs.ctypes.data,
                                      source_rows if source_rows is not None else rows, C.byref(h)), "ttl_q8_upload")
        return Q8(self, h.value, rows, cols)

    def matvec_q8_0(self, w, bias, stage, residual, y):
        _check(self.lib.ttl_matvec_q8_0(self.ctx, w.handle, bias.ptr if bias else None, C.byref(stage),
                                        residual.ptr if residual else None, y.ptr), "ttl_matvec_q8_0")

    def matmul_q8_0(self, w, bias, x, tokens, residual, out, shifts=None):
        """matmul_add_q8_0 for `tokens` rows of x on the device; allocates its workspace.
        shifts: the rows' f16-plane shifts (from rms_norm_rows), for ttl_matmul_q8_0_shifted."""
        ws = self.alloc(max(16, self.lib.ttl_matmul_q8_0_workspace_bytes(tokens, w.cols)))
        try:
            if shifts is None:
                _check(self.lib.ttl_matmul_q8_0(self.ctx, w.handle, bias.ptr if bias else None, x.ptr, tokens,
                                                residual.ptr if residual else None, out.ptr, ws.ptr, ws.nbytes),
                       "ttl_matmul_q8_0")
            else:
                _check(self.lib.ttl_matmul_q8_0_shifted(self.ctx, w.handle, bias.ptr if bias else None, x.ptr,
                                                        shifts.ptr, tokens, residual.ptr if residual else None,
                                                        out.ptr, ws.ptr, ws.nbytes), "ttl_matmul_q8_0_shifted")
            self.sync()
        finally:
            ws.free()

    def rms_norm_rows(self, x, rows, weight, epsilon, out, shifts=None):
        """rms_norm of each of `rows` rows of 2880; shifts (int32 [rows]) receives their
        f16-plane shifts (ttl_rms_norm_rows_shifts)."""
        if shifts is None:
            _check(self.lib.ttl_rms_norm_rows(self.ctx, x.ptr, rows, weight.ptr, epsilon, out.ptr),
                   "ttl_rms_norm_rows")
        else:
            _check(self.lib.ttl_rms_norm_rows_shifts(self.ctx, x.ptr, rows, weight.ptr, epsilon, out.ptr,
                                                     shifts.ptr), "ttl_rms_norm_rows_shifts")

    def attn_qkv(self, qkv, bias, stage, rope, position, capacity, q, kc, vc):
        _check(self.lib.ttl_attn_qkv(self.ctx, qkv.handle, bias.ptr, C.byref(stage), rope.ptr, position.ptr, capacity,
                                     q.ptr, kc.ptr, vc.ptr), "ttl_attn_qkv")

    def attention_decode(self, q, kc, vc, sinks, position, capacity, layer_index, workspace, out):
        _check(self.lib.ttl_attention_decode(self.ctx, q.ptr, kc.ptr, vc.ptr, sinks.ptr, position.ptr, capacity,
                                             layer_index, workspace.ptr, out.ptr), "ttl_attention_decode")

    def attention_decode_noalloc(self, q, kc, vc, sinks, position, capacity, layer_index, out):
        _check(self.lib.ttl_attention_decode_noalloc(self.ctx, q.ptr, kc.ptr, vc.ptr, sinks.ptr, position.ptr,
                                                     capacity, layer_index, out.ptr), "ttl_attention_decode_noalloc")

    def attention_prefill(self, q, kc, vc, sinks, first, tokens, capacity, layer_index, out):
        _check(self.lib.ttl_attention_prefill(self.ctx, q.ptr, kc.ptr, vc.ptr, sinks.ptr, first, tokens, capacity,
                                              layer_index, out.ptr), "ttl_attention_prefill")

    def embedding_q8_0(self, table, vocab, token, out):
        _check(self.lib.ttl_embedding_q8_0(self.ctx, table.ptr, vocab, token.ptr, out.ptr), "ttl_embedding_q8_0")

    def logits_bf16(self, weight, vocab, stage, logits, workspace):
        _check(self.lib.ttl_logits_bf16(self.ctx, weight.ptr, vocab, C.byref(stage), logits.ptr, workspace.ptr),
               "ttl_logits_bf16")

    def logits_q8_0(self, weight, vocab, stage, logits, workspace):
        _check(self.lib.ttl_logits_q8_0(self.ctx, weight.handle, vocab, C.byref(stage), logits.ptr, workspace.ptr),
               "ttl_logits_q8_0")

    def argmax(self, vocab, workspace, token, position=None, history=None, history_len=0):
        _check(self.lib.ttl_argmax(self.ctx, vocab, workspace.ptr, token.ptr, position.ptr if position else None,
                                   history.ptr if history else None, history_len), "ttl_argmax")

    def mxfp8_dequantize(self, x, x_dtype, rows, out):
        _check(self.lib.ttl_mxfp8_dequantize(self.ctx, x.ptr, x_dtype, rows, out.ptr), "ttl_mxfp8_dequantize")

    # ---- graphs ----
    def capture(self, fn):
        """Records the launches fn() makes into a replayable graph."""
        _check(self.lib.ttl_capture_begin(self.ctx), "ttl_capture_begin")
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = self.lib.ttl_capture_end(self.ctx, C.byref(g))
        _check(rc, "ttl_capture_end")
        return Graph(self, g.value)

    # ---- batched prefill (MFMA) ----
    def matmul_mxfp4_selected(self, w, bias, x, x_stride, x_rows, tokens, count, out, expert, workspace=None,
                              mxfp8=False):
        """out[tokens[s]] = W[expert] x[tokens[s]] + bias[expert]; allocates a workspace if none is given.
        mxfp8: the scaled path (activations quantized to MXFP8, v_mfma_scale)."""
        name = "ttl_matmul_mxfp4_selected_mxfp8" if mxfp8 else "ttl_matmul_mxfp4_selected"
        ws = workspace
        if ws is None:
            ws = self.alloc(max(getattr(self.lib, name + "_workspace_bytes")(count), 256))
        try:
            _check(getattr(self.lib, name)(self.ctx, w.handle, bias.ptr if bias else None, x.ptr, x_stride, x_rows,
                                           tokens.ptr, count, out.ptr, expert, ws.ptr, ws.nbytes), name)
            if workspace is None:
                self.sync()
        finally:
            if workspace is None:
                ws.free()

    def moe_prefill_workspace_bytes(self, count, experts, used, x_dtype):
        return self.lib.ttl_moe_prefill_workspace_bytes(count, experts, used, x_dtype)

    def moe_prefill_experts(self, layer, x, x_dtype, count, indices, weights, out, workspace, stages=None):
        if stages is None:
            _check(self.lib.ttl_moe_prefill_experts(self.ctx, C.byref(layer), x.ptr, x_dtype, count, indices.ptr,
                                                    weights.ptr, out.ptr, workspace.ptr, workspace.nbytes),
                   "ttl_moe_prefill_experts")
        else:
            _check(self.lib.ttl_moe_prefill_stages(self.ctx, C.byref(layer), x.ptr, x_dtype, count, indices.ptr,
                                                   weights.ptr, out.ptr, workspace.ptr, workspace.nbytes, stages),
                   "ttl_moe_prefill_stages")

    def moe_prefill_intermediates(self, layer, x_dtype, count, workspace, hidden, down, hidden_scales=None):
        """Each (token, rank) pair's SwiGLU hidden and down row from the workspace of a
        moe_prefill_experts call with the same arguments."""
        _check(self.lib.ttl_moe_prefill_intermediates(self.ctx, C.byref(layer), x_dtype, count, workspace.ptr,
                                                      workspace.nbytes, hidden.ptr, down.ptr,
                                                      hidden_scales.ptr if hidden_scales is not None else None),
               "ttl_moe_prefill_intermediates")

    def moe_prefill(self, layer, x, count, out, indices=None, weights=None, shifts=None, residual=None):
        """GptOssModel::moe_batch on the device (router + experts); allocates its workspace.
        shifts (x's f16-plane shifts) and residual (out = residual + moe) select
        ttl_moe_prefill_fused."""
        ws = self.alloc(self.lib.ttl_moe_prefill_batch_workspace_bytes(count, layer.experts, layer.used))
        try:
            if shifts is None and residual is None:
                _check(self.lib.ttl_moe_prefill(self.ctx, C.byref(layer), x.ptr, count, out.ptr,
                                                indices.ptr if indices else None, weights.ptr if weights else None,
                                                ws.ptr, ws.nbytes), "ttl_moe_prefill")
            else:
                _check(self.lib.ttl_moe_prefill_fused(self.ctx, C.byref(layer), x.ptr,
                                                      shifts.ptr if shifts else None,
                                                      residual.ptr if residual else None, count, out.ptr,
                                                      indices.ptr if indices else None,
                                                      weights.ptr if weights else None, ws.ptr, ws.nbytes),
                       "ttl_moe_prefill_fused")
            self.sync()
        finally:
            ws.free()

    def matvec_mxfp4_experts(self, w, bias, x, x_stride, experts, n, y):
        _check(self.lib.ttl_matvec_mxfp4_experts(self.ctx, w.handle, bias.ptr if bias else None, x.ptr, x_stride,
                                                 experts.ptr, n, y.ptr), "ttl_matvec_mxfp4_experts")
