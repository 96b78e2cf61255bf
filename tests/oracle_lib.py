"""ctypes binding of the CPU oracle (oracle/_build/liborc_oracle.so).

Test infrastructure: the oracle is the parity checker and is never on the
product path.
"""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "liborc_oracle.so")
REF_DRIVER = os.path.join(ROOT, "oracle", "_ref", "ref_driver")

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 14, 30
Q8_0_X8 = 258  # the device's regrouped Q8_0 layout (orc_q8_0_regroup); the oracle reads the GGUF blocks
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}

_fp = C.POINTER(C.c_float)
_ip = C.POINTER(C.c_int32)
_bp = C.POINTER(C.c_uint8)
_lp = C.POINTER(C.c_int64)


def row_bytes(t, n):
    be, bb = BLOCK[t]
    return n // be * bb


def fptr(a):
    return a.ctypes.data_as(_fp)


def iptr(a):
    return a.ctypes.data_as(_ip)


def bptr(a):
    return a.ctypes.data_as(_bp)


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run oracle/Makefile)")
        L = self.L = C.CDLL(path)
        L.orco_fp16.restype = C.c_float
        L.orco_fp16.argtypes = [C.c_uint16]
        L.orco_dequant.argtypes = [C.c_int, _bp, C.c_int64, _fp]
        L.orco_dot.restype = C.c_float
        L.orco_dot.argtypes = [C.c_int, _bp, C.c_int, _fp]
        L.orco_gemv.argtypes = [C.c_int, _bp, C.c_int, C.c_int, _fp, _fp]
        L.orco_gemm.argtypes = [C.c_int, _bp, C.c_int, C.c_int, C.c_int, _fp, _fp]
        L.orco_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_int, C.c_float]
        L.orco_rope.argtypes = [_fp, _fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        L.orco_softmax.argtypes = [_fp, C.c_int]
        L.orco_silu.argtypes = [_fp, C.c_int]
        L.orco_argmax.argtypes = [_fp, C.c_int]
        L.orco_attention.argtypes = [_fp, _fp, _fp, C.c_int, C.c_int, C.c_int, C.c_int, _fp]
        L.orco_model_load.restype = C.c_void_p
        L.orco_model_load.argtypes = [C.c_char_p, C.c_int]
        L.orco_model_free.argtypes = [C.c_void_p]
        L.orco_model_cfg.argtypes = [C.c_void_p, _ip, _fp]
        L.orco_model_reset.argtypes = [C.c_void_p]
        L.orco_model_forward.argtypes = [C.c_void_p, C.c_int32, C.c_int, _fp]
        L.orco_model_forward_batch.argtypes = [C.c_void_p, _ip, C.c_int, C.c_int, _fp]
        L.orco_greedy.argtypes = [C.c_void_p, _ip, C.c_int, C.c_int, _ip]
        L.orco_spec_greedy.argtypes = [C.c_void_p, C.c_void_p, _ip, C.c_int, C.c_int, C.c_int, _ip, _lp]
        L.orco_sampler_new.restype = C.c_void_p
        L.orco_sampler_new.argtypes = [C.c_float, C.c_float, C.c_int, C.c_float, C.c_int, C.c_uint64]
        L.orco_sampler_free.argtypes = [C.c_void_p]
        L.orco_sampler_record.argtypes = [C.c_void_p, C.c_int32]
        L.orco_sampler_sample.restype = C.c_int32
        L.orco_sampler_sample.argtypes = [C.c_void_p, _fp, C.c_int]
        L.orco_mt_next.restype = C.c_uint32
        L.orco_mt_next.argtypes = [C.c_void_p]
        L.orco_sampler_history.argtypes = [C.c_void_p, _ip, C.c_int]
        L.orco_spec_engine.argtypes = [C.c_void_p, C.c_void_p, _ip, C.c_int, C.c_int, C.c_int, C.c_void_p, _ip, _lp]
        L.orco_transform_probs.argtypes = [_fp, C.c_int, _ip, C.c_int, C.c_float, C.c_float, C.c_int, C.c_float, _fp]
        L.orco_accept_resample.restype = C.c_int32
        L.orco_accept_resample.argtypes = [_fp, _fp, C.c_int, C.c_int32, C.c_float, C.c_float, C.POINTER(C.c_int)]
        L.orco_accept_chain.argtypes = [C.c_void_p, _fp, _fp, C.c_int, _ip, C.c_int, C.c_int, _ip,
                                        C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.orco_pick.restype = C.c_int32
        L.orco_pick.argtypes = [_fp, C.c_int, C.c_float]
        L.orco_spec_sampled.argtypes = [C.c_void_p, C.c_void_p, _ip, C.c_int, C.c_int, C.c_int, C.c_void_p, _ip, _lp]

    # codecs / kernels
    def dequant(self, t, raw, n):
        out = np.empty(n, np.float32)
        raw = np.ascontiguousarray(raw, np.uint8)
        assert self.L.orco_dequant(t, bptr(raw), n, fptr(out)) == 0
        return out

    def gemv(self, t, w, n_out, n_in, x):
        y = np.empty(n_out, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        assert self.L.orco_gemv(t, bptr(w), n_out, n_in, fptr(x), fptr(y)) == 0
        return y

    def gemm(self, t, w, n_tok, n_out, n_in, X):
        Y = np.empty((n_tok, n_out), np.float32)
        X = np.ascontiguousarray(X, np.float32)
        assert self.L.orco_gemm(t, bptr(w), n_tok, n_out, n_in, fptr(X), fptr(Y)) == 0
        return Y

    def rmsnorm(self, x, w, eps=1e-5):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.empty_like(x)
        self.L.orco_rmsnorm(fptr(out), fptr(x), fptr(w), x.size, eps)
        return out

    def rope(self, q, k, H, KVH, hd, pos, base):
        q = np.array(q, np.float32)
        k = np.array(k, np.float32)
        self.L.orco_rope(fptr(q), fptr(k), H, KVH, hd, pos, base)
        return q, k

    def softmax(self, x):
        x = np.array(x, np.float32)
        self.L.orco_softmax(fptr(x), x.size)
        return x

    def silu(self, x):
        x = np.array(x, np.float32)
        self.L.orco_silu(fptr(x), x.size)
        return x

    def argmax(self, x):
        x = np.ascontiguousarray(x, np.float32)
        return self.L.orco_argmax(fptr(x), x.size)

    def attention(self, q, kc, vc, H, KVH, hd, pos):
        out = np.zeros(H * hd, np.float32)
        q, kc, vc = (np.ascontiguousarray(a, np.float32) for a in (q, kc, vc))
        self.L.orco_attention(fptr(q), fptr(kc), fptr(vc), H, KVH, hd, pos, fptr(out))
        return out


class OracleModel:
    def __init__(self, orc: Oracle, path, ctx_len=512):
        self.o = orc
        self.h = orc.L.orco_model_load(path.encode(), ctx_len)
        if not self.h:
            raise RuntimeError(f"oracle could not load {path}")
        cfg = np.zeros(10, np.int32)
        rope = C.c_float()
        orc.L.orco_model_cfg(self.h, iptr(cfg), C.byref(rope))
        (self.n_vocab, self.n_layers, self.n_heads, self.n_kv_heads, self.embed_dim, self.ffn, self.head_dim,
         self.ctx_len, self.has_bias, self.tied) = (int(v) for v in cfg)
        self.rope = rope.value

    def __del__(self):
        if getattr(self, "h", None):
            self.o.L.orco_model_free(self.h)
            self.h = None

    def reset(self):
        self.o.L.orco_model_reset(self.h)

    def forward(self, tok, pos, logits=True):
        out = np.empty(self.n_vocab, np.float32) if logits else None
        rc = self.o.L.orco_model_forward(self.h, tok, pos, fptr(out) if logits else None)
        assert rc == 0
        return out

    def forward_batch(self, toks, start_pos, logits=True):
        toks = np.ascontiguousarray(toks, np.int32)
        out = np.empty((toks.size, self.n_vocab), np.float32) if logits else None
        rc = self.o.L.orco_model_forward_batch(self.h, iptr(toks), toks.size, start_pos, fptr(out) if logits else None)
        assert rc == 0
        return out

    def greedy(self, prompt, n_gen):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_gen, np.int32)
        n = self.o.L.orco_greedy(self.h, iptr(prompt), prompt.size, n_gen, iptr(out))
        return out[:n]

    def spec_greedy(self, draft, prompt, n_gen, k):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_gen + k + 2, np.int32)
        st = np.zeros(3, np.int64)
        n = self.o.L.orco_spec_greedy(self.h, draft.h, iptr(prompt), prompt.size, n_gen, k, iptr(out),
                                      st.ctypes.data_as(_lp))
        return out[:n], {"accepted": int(st[0]), "proposed": int(st[1]), "passes": int(st[2])}

    def spec_sampled(self, draft, prompt, n_gen, k, temperature=0.8, top_p=0.95, top_k=40, repeat_penalty=1.1,
                     repeat_last=64, seed=42):
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_gen + k + 2, np.int32)
        st = np.zeros(3, np.int64)
        s = self.o.L.orco_sampler_new(temperature, top_p, top_k, repeat_penalty, repeat_last, seed)
        n = self.o.L.orco_spec_sampled(self.h, draft.h, iptr(prompt), prompt.size, n_gen, k, s, iptr(out),
                                       st.ctypes.data_as(_lp))
        self.o.L.orco_sampler_free(s)
        return out[:n], {"accepted": int(st[0]), "proposed": int(st[1]), "passes": int(st[2])}
