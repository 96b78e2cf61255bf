"""ctypes binding of the C ABI in include/orc.h (liborc_hip.so) and of the
host C API in include/oracle_host.h (liboracle_host.so).

Used by tests/, bench.py and __graft_entry__.py. Loading fails loudly when the
HIP library has not been built: there is no CPU fallback on the product path.
"""
import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG, "lib")
HIP_LIB = os.path.join(LIB_DIR, "liborc_hip.so")
HOST_LIB = os.path.join(LIB_DIR, "liboracle_host.so")
BIN_DIR = os.path.join(PKG, "bin")

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
EPI_STORE, EPI_ACCUM, EPI_SWIGLU = 0, 1, 2
Q8_0_X8 = 258  # ORC_Q8_0_X8: Q8_0 regrouped by orc_q8_0_regroup

_vp = C.c_void_p
_fp = C.POINTER(C.c_float)
_ip = C.POINTER(C.c_int32)


class OrcError(RuntimeError):
    pass


class Seg(C.Structure):
    _fields_ = [("d_w", _vp), ("n_out", C.c_int), ("d_y", _vp), ("d_bias", _vp)]


# (name, restype, argtypes) for every entry point declared in include/orc.h
ABI = [
    ("orc_init", C.c_int, [C.c_int]),
    ("orc_shutdown", C.c_int, []),
    ("orc_last_error", C.c_char_p, []),
    ("orc_device_info", C.c_int, [C.c_char_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_size_t)]),
    ("orc_malloc", C.c_int, [C.POINTER(_vp), C.c_size_t]),
    ("orc_free", C.c_int, [_vp]),
    ("orc_memcpy_h2d", C.c_int, [_vp, _vp, C.c_size_t, _vp]),
    ("orc_memcpy_d2h", C.c_int, [_vp, _vp, C.c_size_t, _vp]),
    ("orc_memcpy_d2d", C.c_int, [_vp, _vp, C.c_size_t, _vp]),
    ("orc_fill", C.c_int, [_vp, C.c_int, C.c_size_t, _vp]),
    ("orc_upload", C.c_int, [_vp, C.c_size_t, C.POINTER(_vp)]),
    ("orc_stream_create", C.c_int, [C.POINTER(_vp)]),
    ("orc_stream_destroy", C.c_int, [_vp]),
    ("orc_stream_sync", C.c_int, [_vp]),
    ("orc_device_sync", C.c_int, []),
    ("orc_graph_begin", C.c_int, [_vp]),
    ("orc_graph_end", C.c_int, [_vp, C.POINTER(_vp)]),
    ("orc_graph_launch", C.c_int, [_vp, _vp]),
    ("orc_graph_destroy", C.c_int, [_vp]),
    ("orc_event_create", C.c_int, [C.POINTER(_vp)]),
    ("orc_event_destroy", C.c_int, [_vp]),
    ("orc_event_record", C.c_int, [_vp, _vp]),
    ("orc_event_elapsed_ms", C.c_int, [_vp, _vp, C.POINTER(C.c_float)]),
    ("orc_row_bytes", C.c_int64, [C.c_int, C.c_int64]),
    ("orc_q8_0_regroup", C.c_int, [_vp, C.c_int64, _vp]),
    ("orc_dequant", C.c_int, [C.c_int, _vp, C.c_int64, _vp, _vp]),
    ("orc_embed", C.c_int, [C.c_int, _vp, C.c_int, C.c_int, _vp, C.c_int, _vp, C.c_int, _vp]),
    ("orc_gemm", C.c_int, [C.c_int, _vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp, C.c_int, _vp]),
    ("orc_gemm_fused", C.c_int, [C.c_int, C.POINTER(Seg), C.c_int, C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp,
                                 C.c_float, C.c_int, _vp]),
    ("orc_gemm_fused_mixed", C.c_int, [_ip, C.POINTER(Seg), C.c_int, C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp,
                                       C.c_float, C.c_int, _vp]),
    ("orc_rmsnorm", C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_float, _vp]),
    ("orc_qk_norm", C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, C.c_float, _vp]),
    ("orc_rope_kv_store", C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp,
                                    C.c_int, _vp]),
    ("orc_rope_kv_store_at", C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp,
                                       _vp, C.c_int, _vp]),
    ("orc_attn_workspace", C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int]),
    ("orc_attn_gqa", C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, C.c_int, _vp,
                               C.c_int, _vp, _vp]),
    ("orc_attn_gqa_at", C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp,
                                  C.c_int, _vp, C.c_int, _vp, _vp]),
    ("orc_attn_fused_workspace", C.c_size_t, [C.c_int, C.c_int, C.c_int]),
    ("orc_attn_wg_limit", C.c_int, []),
    ("orc_attn_prefill", C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, C.c_int,
                                   _vp, C.c_int, _vp]),
    ("orc_attn_fused_at", C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp, _vp,
                                    C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp]),
    ("orc_argmax_workspace", C.c_size_t, [C.c_int, C.c_int]),
    ("orc_argmax", C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp]),
    ("orc_argmax_noalloc", C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    ("orc_spec_accept_greedy", C.c_int, [_vp, _vp, C.c_int, _vp, _vp]),
    ("orc_spec_accept_greedy_at", C.c_int, [_vp, _vp, C.c_int, _vp, _vp, _vp, _vp]),
    ("orc_decode_advance", C.c_int, [_vp, _vp, _vp, _vp, _vp]),
    ("orc_sampler_state_bytes", C.c_size_t, []),
    ("orc_sampler_init", C.c_int, [_vp, C.c_float, C.c_float, C.c_int, C.c_float, C.c_int, C.c_uint64, _vp, C.c_int,
                                   _vp]),
    ("orc_sample", C.c_int, [_vp, _vp, C.c_int, _vp, _vp]),
    ("orc_sampler_record", C.c_int, [_vp, _vp, C.c_int, _vp]),
    ("orc_sampler_history", C.c_int, [_vp, _vp, C.c_int, _vp, _vp]),
    ("orc_spec_accept_engine", C.c_int, [_vp, _vp, C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp,
                                         _vp]),
    ("orc_transform_probs", C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp, C.c_int, _vp]),
    ("orc_draw", C.c_int, [_vp, _vp, C.c_int, _vp, _vp, _vp]),
    ("orc_transform_draw", C.c_int, [_vp, _vp, C.c_int, _vp, C.c_int, _vp, _vp, _vp, _vp]),
    ("orc_accept_resample", C.c_int, [_vp, _vp, C.c_int, C.c_int32, C.c_float, C.c_float, _vp, _vp]),
    ("orc_spec_accept_stochastic", C.c_int, [_vp, _vp, C.c_int, _vp, C.c_int, C.c_int, _vp, C.c_int, C.c_int, _vp,
                                             _vp, _vp, _vp, _vp]),
    ("orc_sampler_set_params", C.c_int, [_vp, C.c_float, C.c_float, C.c_int, C.c_float, C.c_int, _vp]),
    ("orc_sampler_clear_history", C.c_int, [_vp, _vp]),
    ("orc_vec_binary", C.c_int, [C.c_int, _vp, _vp, _vp, C.c_int, _vp]),
    ("orc_vec_silu", C.c_int, [_vp, C.c_int, _vp]),
    ("orc_softmax", C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp]),
    ("orc_dot", C.c_int, [_vp, _vp, C.c_int, _vp, _vp]),
    ("orc_matmul_f32", C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp]),
    ("orc_rope_pos", C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    ("orc_prof_enable", C.c_int, [C.c_int]),
    ("orc_prof_accumulate", C.c_int, []),
    ("orc_prof_read", C.c_int, [C.c_int, C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_double),
                                C.POINTER(C.c_double)]),
]


def load_hip_lib(path=HIP_LIB):
    if not os.path.exists(path):
        raise OrcError(f"{path} is missing: build it with __graft_entry__.build() (no CPU fallback exists)")
    lib = C.CDLL(path, mode=C.RTLD_GLOBAL)
    for name, res, args in ABI:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


class Device:
    """The HIP library plus small helpers for device buffers."""

    def __init__(self, device=0):
        self.L = load_hip_lib()
        self.check(self.L.orc_init(device))

    def check(self, rc):
        if rc != 0:
            raise OrcError(f"orc error {rc}: {self.L.orc_last_error().decode()}")
        return rc

    def info(self):
        name = C.create_string_buffer(256)
        cu = C.c_int()
        hbm = C.c_size_t()
        self.check(self.L.orc_device_info(name, 256, C.byref(cu), C.byref(hbm)))
        return name.value.decode(), cu.value, hbm.value

    def alloc(self, nbytes):
        p = _vp()
        self.check(self.L.orc_malloc(C.byref(p), max(int(nbytes), 1)))
        return DBuf(self, p.value, int(nbytes))

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes)
        b.write(arr)
        return b

    def sync(self):
        self.check(self.L.orc_device_sync())


class DBuf:
    def __init__(self, dev, ptr, nbytes):
        self.dev, self.ptr, self.nbytes = dev, ptr, nbytes

    def write(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        self.dev.check(self.dev.L.orc_memcpy_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes, None))

    def read(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        self.dev.check(self.dev.L.orc_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes, None))
        return out

    def at(self, offset):
        return self.ptr + offset

    def free(self):
        if self.ptr:
            self.dev.L.orc_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ── host API (include/oracle_host.h) ─────────────────────────────────────────
HOST_ABI = [
    ("orch_load", _vp, [C.c_char_p, C.c_int]),
    ("orch_free", None, [_vp]),
    ("orch_error", C.c_char_p, [_vp]),
    ("orch_cfg", C.c_int, [_vp, _ip, _fp]),
    ("orch_reset", C.c_int, [_vp]),
    ("orch_forward", C.c_int, [_vp, C.c_int32, C.c_int, _fp]),
    ("orch_forward_batch", C.c_int, [_vp, _ip, C.c_int, C.c_int, _fp]),
    ("orch_greedy", C.c_int, [_vp, _ip, C.c_int, C.c_int, _ip, C.c_int]),
    ("orch_spec_greedy", C.c_int, [_vp, _vp, _ip, C.c_int, C.c_int, C.c_int, _ip, C.POINTER(C.c_int64), C.c_int]),
    ("orch_spec_engine", C.c_int, [_vp, _vp, _ip, C.c_int, C.c_int, C.c_int, _fp, _ip, C.c_uint64, _ip,
                                   C.POINTER(C.c_int64)]),
    ("orch_spec_sampled", C.c_int, [_vp, _vp, _ip, C.c_int, C.c_int, C.c_int, _fp, _ip, C.c_uint64, _ip,
                                    C.POINTER(C.c_int64)]),
    ("orch_set_graphs", C.c_int, [C.c_int]),
    ("orch_weight_bytes", C.c_double, [_vp, C.c_int]),
    ("orch_sync", C.c_int, []),
    ("orch_gguf_device_type", C.c_int, [_vp, C.c_char_p]),
    ("orch_gguf_gemm", C.c_int, [_vp, C.c_char_p, _fp, C.c_int, C.c_int, C.c_int, _fp]),
    ("orch_gguf_dequant_row", C.c_int, [_vp, C.c_char_p, C.c_int64, _fp]),
    ("orch_embed_tokens", C.c_int, [_vp, _ip, C.c_int, _fp]),
    ("orch_save_state", C.c_int, [_vp, C.c_char_p, C.c_int]),
    ("orch_load_state", C.c_int, [_vp, C.c_char_p, _ip]),
    ("orch_snapshot_kv", _vp, [_vp, C.c_int]),
    ("orch_restore_kv", C.c_int, [_vp, _vp]),
    ("orch_snapshot_pos", C.c_int, [_vp]),
    ("orch_snapshot_free", None, [_vp]),
    ("orch_norm_cache_matches", C.c_int, [_vp]),
    ("orch_ops_rmsnorm", None, [_fp, _fp, _fp, C.c_int, C.c_float]),
    ("orch_ops_matmul", None, [_fp, _fp, _fp, C.c_int, C.c_int, C.c_int]),
    ("orch_ops_matmul_nn", None, [_fp, _fp, _fp, C.c_int, C.c_int, C.c_int]),
    ("orch_ops_silu", None, [_fp, C.c_int]),
    ("orch_ops_mul", None, [_fp, _fp, _fp, C.c_int]),
    ("orch_ops_add", None, [_fp, _fp, C.c_int]),
    ("orch_ops_copy", None, [_fp, _fp, C.c_int]),
    ("orch_ops_softmax", None, [_fp, C.c_int]),
    ("orch_ops_rope", None, [_fp, _fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
    ("orch_ops_argmax", C.c_int, [_fp, C.c_int]),
    ("orch_ops_dot", C.c_float, [_fp, _fp, C.c_int]),
    ("orch_engine_new", _vp, [C.c_char_p, C.c_char_p]),
    ("orch_engine_free", None, [_vp]),
    ("orch_engine_error", C.c_char_p, [_vp]),
    ("orch_engine_set_seed", None, [_vp, C.c_uint64]),
    ("orch_engine_generate", C.c_int64, [_vp, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), C.c_int, C.c_int,
                                         C.c_float, C.c_float, C.c_float, C.c_int, C.POINTER(C.c_uint8),
                                         C.c_int64]),
    ("orch_engine_embed", C.c_int, [_vp, C.c_char_p, _fp]),
    ("orch_tokenizer_load", _vp, [C.c_char_p]),
    ("orch_tokenizer_free", None, [_vp]),
    ("orch_tok_encode", C.c_int, [_vp, C.c_char_p, C.c_int64, C.c_int, _ip, C.c_int]),
    ("orch_tok_decode_one", C.c_int, [_vp, C.c_int32, C.c_char_p, C.c_int]),
    ("orch_tok_special_id", C.c_int32, [_vp, C.c_char_p]),
    ("orch_tok_bos_eos", C.c_int32, [_vp, C.c_int]),
    ("orch_sampler_new", _vp, [C.c_float, C.c_float, C.c_int, C.c_float, C.c_int, C.c_uint64]),
    ("orch_sampler_free", None, [_vp]),
    ("orch_sampler_sample", C.c_int32, [_vp, _fp, C.c_int]),
    ("orch_sampler_record", None, [_vp, C.c_int32]),
    ("orch_sampler_reset", None, [_vp]),
    ("orch_sampler_set_params", None, [_vp, C.c_float, C.c_float, C.c_int, C.c_float, C.c_int]),
]

_host = None


def load_host_lib(path=HOST_LIB):
    global _host
    if _host is None:
        load_hip_lib()  # resolves liborc_hip.so first (and fails loudly if missing)
        if not os.path.exists(path):
            raise OrcError(f"{path} is missing: build it with __graft_entry__.build()")
        lib = C.CDLL(path)
        for name, res, args in HOST_ABI:
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _host = lib
    return _host


def _i32(a):
    return np.ascontiguousarray(a, np.int32)


class Model:
    """Device-resident model (Model API of core/model.hpp) through liboracle_host."""

    def __init__(self, path, ctx_len=0):
        self.L = load_host_lib()
        self.h = self.L.orch_load(str(path).encode(), int(ctx_len))
        if not self.h:
            raise OrcError(f"cannot load {path}: {self.L.orch_error(None).decode()}")
        cfg = np.zeros(10, np.int32)
        rope = C.c_float()
        self.L.orch_cfg(self.h, cfg.ctypes.data_as(_ip), C.byref(rope))
        (self.n_vocab, self.n_layers, self.n_heads, self.n_kv_heads, self.embed_dim, self.ffn, self.head_dim,
         self.ctx_len, self.has_bias, self.tied) = (int(v) for v in cfg)
        self.rope = rope.value

    def close(self):
        if getattr(self, "h", None):
            self.L.orch_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc < 0:
            raise OrcError(f"host error {rc}: {self.L.orch_error(self.h).decode()}")
        return rc

    def reset(self):
        self._check(self.L.orch_reset(self.h))

    def forward(self, tok, pos, logits=True):
        out = np.empty(self.n_vocab, np.float32) if logits else None
        self._check(self.L.orch_forward(self.h, int(tok), int(pos), out.ctypes.data_as(_fp) if logits else None))
        return out

    def forward_batch(self, toks, start_pos, logits=True):
        toks = _i32(toks)
        out = np.empty((toks.size, self.n_vocab), np.float32) if logits else None
        self._check(self.L.orch_forward_batch(self.h, toks.ctypes.data_as(_ip), toks.size, int(start_pos),
                                              out.ctypes.data_as(_fp) if logits else None))
        return out

    def greedy(self, prompt, n_gen, prefill=True):
        prompt = _i32(prompt)
        out = np.empty(n_gen, np.int32)
        n = self._check(self.L.orch_greedy(self.h, prompt.ctypes.data_as(_ip), prompt.size, n_gen,
                                           out.ctypes.data_as(_ip), int(prefill)))
        return out[:n]

    def spec_greedy(self, draft, prompt, n_gen, k, prefill=True):
        prompt = _i32(prompt)
        out = np.empty(n_gen + k + 2, np.int32)
        st = np.zeros(4, np.int64)
        n = self._check(self.L.orch_spec_greedy(self.h, draft.h, prompt.ctypes.data_as(_ip), prompt.size, n_gen, k,
                                                out.ctypes.data_as(_ip), st.ctypes.data_as(C.POINTER(C.c_int64)),
                                                int(prefill)))
        return out[:n], {"accepted": int(st[0]), "proposed": int(st[1]), "passes": int(st[2]), "rounds": int(st[3])}

    def spec_engine(self, draft, prompt, n_gen, k, temperature=0.8, top_p=0.95, top_k=40, repeat_penalty=1.1,
                    repeat_last=64, seed=42):
        """Engine-style stochastic speculative decode (core/engine.cpp:100-240) on the device."""
        prompt = _i32(prompt)
        out = np.empty(n_gen + k + 2, np.int32)
        st = np.zeros(3, np.int64)
        fs = np.array([temperature, top_p, repeat_penalty], np.float32)
        iv = np.array([top_k, repeat_last], np.int32)
        n = self._check(self.L.orch_spec_engine(self.h, draft.h, prompt.ctypes.data_as(_ip), prompt.size, n_gen, k,
                                                fs.ctypes.data_as(_fp), iv.ctypes.data_as(_ip), int(seed),
                                                out.ctypes.data_as(_ip), st.ctypes.data_as(C.POINTER(C.c_int64))))
        return out[:n], {"accepted": int(st[0]), "proposed": int(st[1]), "passes": int(st[2])}

    def spec_sampled(self, draft, prompt, n_gen, k, temperature=0.8, top_p=0.95, top_k=40, repeat_penalty=1.1,
                     repeat_last=64, seed=42):
        """Speculative sampling (min(1, p/q) acceptance, residual resampling) on the device."""
        prompt = _i32(prompt)
        out = np.empty(n_gen + k + 2, np.int32)
        st = np.zeros(3, np.int64)
        fs = np.array([temperature, top_p, repeat_penalty], np.float32)
        iv = np.array([top_k, repeat_last], np.int32)
        n = self._check(self.L.orch_spec_sampled(self.h, draft.h, prompt.ctypes.data_as(_ip), prompt.size, n_gen, k,
                                                 fs.ctypes.data_as(_fp), iv.ctypes.data_as(_ip), int(seed),
                                                 out.ctypes.data_as(_ip), st.ctypes.data_as(C.POINTER(C.c_int64))))
        return out[:n], {"accepted": int(st[0]), "proposed": int(st[1]), "passes": int(st[2])}

    def weight_bytes(self, logits=True):
        return self.L.orch_weight_bytes(self.h, int(logits))

    # GGUFParser drop-ins of this model (model.gguf().gemv_q / gemm_q / dequantize_row)
    def gguf_device_type(self, tensor):
        return self.L.orch_gguf_device_type(self.h, tensor.encode())

    def gguf_gemv(self, tensor, x, j0=0, j1=None, n_out=None):
        x = np.ascontiguousarray(x, np.float32)
        j1 = n_out if j1 is None else j1
        out = np.zeros(j1, np.float32)
        self._check(self.L.orch_gguf_gemm(self.h, tensor.encode(), x.ctypes.data_as(_fp), 1, int(j0), int(j1),
                                          out.ctypes.data_as(_fp)))
        return out[j0:]

    def gguf_gemm(self, tensor, X, n_out):
        X = np.ascontiguousarray(X, np.float32)
        out = np.zeros((X.shape[0], n_out), np.float32)
        self._check(self.L.orch_gguf_gemm(self.h, tensor.encode(), X.ctypes.data_as(_fp), X.shape[0], 0, int(n_out),
                                          out.ctypes.data_as(_fp)))
        return out

    def gguf_dequant_row(self, tensor, row, n_in):
        out = np.zeros(n_in, np.float32)
        self._check(self.L.orch_gguf_dequant_row(self.h, tensor.encode(), int(row), out.ctypes.data_as(_fp)))
        return out

    def embed_tokens(self, tokens):
        """Model::embed_tokens (core/model.cpp:248-270)."""
        t = _i32(tokens)
        out = np.zeros(self.embed_dim, np.float32)
        self._check(self.L.orch_embed_tokens(self.h, t.ctypes.data_as(_ip), t.size, out.ctypes.data_as(_fp)))
        return out

    def save_state(self, path, pos):
        """Model::save_state (core/model.cpp:156-181): the .orkv file."""
        self._check(self.L.orch_save_state(self.h, str(path).encode(), int(pos)))

    def load_state(self, path):
        """Model::load_state (core/model.cpp:184-236); the saved position, or
        None if the file is missing or incompatible (the reference's false)."""
        pos = C.c_int(-1)
        rc = self.L.orch_load_state(self.h, str(path).encode(), C.cast(C.pointer(pos), _ip))
        return None if rc else pos.value

    def snapshot_kv(self, pos):
        """Model::snapshot_kv (core/model.hpp:104): a device copy of the KV cache."""
        h = self.L.orch_snapshot_kv(self.h, int(pos))
        if not h:
            raise OrcError("snapshot_kv failed")
        return KVSnapshot(self.L, h)

    def restore_kv(self, snap):
        self._check(self.L.orch_restore_kv(self.h, snap.h))

    def norm_cache_matches(self):
        return bool(self.L.orch_norm_cache_matches(self.h))


class KVSnapshot:
    def __init__(self, L, h):
        self.L, self.h = L, h

    @property
    def pos(self):
        return self.L.orch_snapshot_pos(self.h)

    def __del__(self):
        if getattr(self, "h", None):
            self.L.orch_snapshot_free(self.h)
            self.h = None


class Sampler:
    """Sampler (core/sampler.hpp:24-48) on a device state, host logits."""

    def __init__(self, temperature=0.7, top_p=0.9, top_k=40, repeat_pen=1.1, repeat_last=64, seed=42):
        self.L = load_host_lib()
        self.h = self.L.orch_sampler_new(temperature, top_p, int(top_k), repeat_pen, int(repeat_last), int(seed))
        if not self.h:
            raise OrcError("Sampler: device state could not be created")

    def sample(self, logits):
        """Next id; the array is rewritten in place as the reference's is."""
        assert logits.dtype == np.float32 and logits.flags.c_contiguous
        return int(self.L.orch_sampler_sample(self.h, logits.ctypes.data_as(_fp), logits.size))

    def record(self, tok):
        self.L.orch_sampler_record(self.h, int(tok))

    def reset(self):
        self.L.orch_sampler_reset(self.h)

    def set_params(self, temperature, top_p, top_k, repeat_pen, repeat_last):
        self.L.orch_sampler_set_params(self.h, temperature, top_p, int(top_k), repeat_pen, int(repeat_last))

    def __del__(self):
        if getattr(self, "h", None):
            self.L.orch_sampler_free(self.h)
            self.h = None


def split_pieces(buf):
    """(uint32 length, bytes) records -> list of bytes."""
    out, i = [], 0
    while i < len(buf):
        n = int.from_bytes(buf[i:i + 4], "little")
        out.append(bytes(buf[i + 4:i + 4 + n]))
        i += 4 + n
    return out


class Tokenizer:
    """Tokenizer (core/tokenizer.hpp:17-44) from a GGUF's metadata; host only."""

    def __init__(self, path):
        self.L = load_host_lib()
        self.h = self.L.orch_tokenizer_load(str(path).encode())
        if not self.h:
            raise OrcError(f"cannot load a tokenizer from {path}")

    def encode(self, text, add_bos=True):
        b = text if isinstance(text, bytes) else text.encode()
        out = np.zeros(len(b) + 8, np.int32)
        n = self.L.orch_tok_encode(self.h, b, len(b), int(add_bos), out.ctypes.data_as(_ip), out.size)
        if n < 0:
            raise OrcError("encode failed")
        return out[:n].copy()

    def decode_one(self, tok):
        buf = C.create_string_buffer(256)
        n = self.L.orch_tok_decode_one(self.h, int(tok), buf, 256)
        if n > 256:
            buf = C.create_string_buffer(n)
            n = self.L.orch_tok_decode_one(self.h, int(tok), buf, n)
        return buf.raw[:n]

    def special_id(self, name):
        return int(self.L.orch_tok_special_id(self.h, name.encode()))

    def bos_eos(self):
        return int(self.L.orch_tok_bos_eos(self.h, 0)), int(self.L.orch_tok_bos_eos(self.h, 1))

    def __del__(self):
        if getattr(self, "h", None):
            self.L.orch_tokenizer_free(self.h)
            self.h = None


class Engine:
    """Engine (core/engine.hpp:35-76) on the device path."""

    def __init__(self, model_path, draft_path=None, seed=None):
        self.L = load_host_lib()
        self.h = self.L.orch_engine_new(str(model_path).encode(), str(draft_path).encode() if draft_path else None)
        if not self.h:
            raise OrcError(f"engine load failed: {self.L.orch_engine_error(None).decode()}")
        if seed is not None:
            self.L.orch_engine_set_seed(self.h, int(seed))

    def generate(self, messages, n_predict=256, temperature=0.7, top_p=0.9, repeat_penalty=1.15, repeat_last_n=64):
        """The on_token pieces (bytes) in order; their concatenation is the reply."""
        roles = (C.c_char_p * len(messages))(*[r.encode() for r, _ in messages])
        conts = (C.c_char_p * len(messages))(*[c.encode() for _, c in messages])
        cap = 64 * (n_predict + 16) + 4096
        buf = (C.c_uint8 * cap)()
        n = self.L.orch_engine_generate(self.h, roles, conts, len(messages), n_predict, temperature, top_p,
                                        repeat_penalty, repeat_last_n, buf, cap)
        if n < 0:
            raise OrcError(f"generate failed: {self.L.orch_engine_error(self.h).decode()}")
        return split_pieces(bytes(buf)[:n])

    def embed(self, text, dim):
        out = np.zeros(dim, np.float32)
        if self.L.orch_engine_embed(self.h, text.encode(), out.ctypes.data_as(_fp)):
            raise OrcError("embed failed")
        return out

    def close(self):
        if getattr(self, "h", None):
            self.L.orch_engine_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


class HostOps:
    """namespace ops (core/ops.hpp:42-92) on numpy float32 arrays, through
    liboracle_host (computed on the GPU)."""

    def __init__(self):
        self.L = load_host_lib()

    @staticmethod
    def _p(a):
        assert a.dtype == np.float32 and a.flags.c_contiguous
        return a.ctypes.data_as(_fp)

    def rmsnorm(self, x, w, eps=1e-5):
        out = np.empty_like(x)
        self.L.orch_ops_rmsnorm(self._p(out), self._p(x), self._p(w), x.size, eps)
        return out

    def matmul(self, a, b, nn=False):
        m, k = a.shape
        n = b.shape[1] if nn else b.shape[0]
        out = np.empty((m, n), np.float32)
        (self.L.orch_ops_matmul_nn if nn else self.L.orch_ops_matmul)(self._p(out), self._p(a), self._p(b), m, n, k)
        return out

    def silu(self, x):
        x = x.copy()
        self.L.orch_ops_silu(self._p(x), x.size)
        return x

    def mul(self, a, b):
        out = np.empty_like(a)
        self.L.orch_ops_mul(self._p(out), self._p(a), self._p(b), a.size)
        return out

    def add(self, a, b):
        a = a.copy()
        self.L.orch_ops_add(self._p(a), self._p(b), a.size)
        return a

    def copy(self, a):
        out = np.empty_like(a)
        self.L.orch_ops_copy(self._p(out), self._p(a), a.size)
        return out

    def softmax(self, x):
        x = x.copy()
        self.L.orch_ops_softmax(self._p(x), x.size)
        return x

    def rope(self, q, k, n_heads, n_kv, hd, pos, base):
        q, k = q.copy(), k.copy()
        self.L.orch_ops_rope(self._p(q), self._p(k), n_heads, n_kv, hd, pos, base)
        return q, k

    def argmax(self, x):
        return int(self.L.orch_ops_argmax(self._p(x), x.size))

    def dot(self, a, b):
        return float(self.L.orch_ops_dot(self._p(a), self._p(b), a.size))
