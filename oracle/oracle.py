"""ctypes bindings for the parity checkers. TEST INFRASTRUCTURE ONLY.

Two checkers live under oracle/:
  * ``Oracle``  -- the C restatement (mmf_oracle.c -> _build/libmmf_oracle.so);
  * ``Ref``     -- the reference engine compiled from its own sources plus ref_harness.cpp
                  (-> _ref/libmmfree_ref.so), present where /root/reference was when the
                  checkers were built.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libmmf_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libmmfree_ref.so")
REF_CLI = os.path.join(HERE, "_ref", "mmfree-cli")

FLOAT, FIXED, INT8 = 0, 1, 2

_fp = C.POINTER(C.c_float)
_i8p = C.POINTER(C.c_int8)
_i32p = C.POINTER(C.c_int32)
_i64p = C.POINTER(C.c_int64)
_szp = C.POINTER(C.c_size_t)


def _p(a, t):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the checkers must be contiguous"
    return a.ctypes.data_as(t)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class MoLayer(C.Structure):
    _fields_ = [("attn_norm", _fp), ("mlp_norm", _fp), ("g_norm", _fp),
                ("wq", _i8p * 6), ("scale_w", C.c_float * 6), ("normw", _fp * 6)]


class MoModel(C.Structure):
    _fields_ = [("V", C.c_size_t), ("H", C.c_size_t), ("L", C.c_size_t), ("I", C.c_size_t),
                ("eps", C.c_float), ("use_lower_bound", C.c_int), ("emb", _fp), ("norm_w", _fp),
                ("lm_wq", _i8p), ("lm_scale_w", C.c_float), ("lm_normw", _fp),
                ("lower_bounds", _fp), ("layers", C.POINTER(MoLayer))]


class Oracle:
    """The C restatement of the reference numerics (see mmf_oracle.h)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run `make -C oracle`)")
        L = self.lib = C.CDLL(path)
        L.mo_sumsq.restype = C.c_float
        L.mo_sumsq.argtypes = [_fp, C.c_size_t]
        L.mo_hsum8.restype = C.c_float
        L.mo_hsum8.argtypes = [_fp]
        L.mo_ternary_dot_f32.restype = C.c_float
        L.mo_ternary_dot_f32.argtypes = [_fp, _i8p, C.c_size_t]
        L.mo_exp_body.restype = C.c_float
        L.mo_exp_body.argtypes = [C.c_float]
        L.mo_exp_tail.restype = C.c_float
        L.mo_exp_tail.argtypes = [C.c_float]
        L.mo_rstd.restype = C.c_float
        L.mo_rstd.argtypes = [C.c_float, C.c_size_t, C.c_float]
        for n in ("mo_sigmoid", "mo_silu"):
            getattr(L, n).argtypes = [_fp, _fp, C.c_size_t]
        L.mo_swiglu.argtypes = [_fp, _fp, _fp, C.c_size_t]
        L.mo_quant_q510.argtypes = [_i32p, _fp, C.c_float, C.c_size_t]
        L.mo_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_size_t, C.c_size_t, C.c_float]
        L.mo_rmsnorm_swishgate.argtypes = [_fp, _fp, _fp, _fp, C.c_size_t, C.c_size_t, C.c_float]
        L.mo_hgrn_scan.argtypes = [_fp, _fp, _fp, C.c_size_t, C.c_size_t, _fp]
        L.mo_bitlinear.argtypes = [_fp, _fp, _fp, _i8p, C.c_float, C.c_size_t, C.c_size_t,
                                   C.c_size_t, C.c_float, C.c_int, C.c_int, _fp, _i32p, _i32p, _fp]
        L.mo_ternary_matmul.argtypes = [_i32p, _i32p, _i8p, C.c_size_t, C.c_size_t, C.c_size_t]
        L.mo_block.argtypes = [C.POINTER(MoModel), C.c_int, C.c_int, _fp, C.c_size_t, C.c_size_t,
                               _fp, C.c_int, _fp]
        L.mo_generate.restype = C.c_size_t
        L.mo_generate.argtypes = [C.POINTER(MoModel), C.c_int, C.c_int, _i64p, C.c_size_t,
                                  C.c_size_t, C.c_int64, _i64p, _fp, _fp]
        L.mo_forward.argtypes = [C.POINTER(MoModel), C.c_int, C.c_int, _i64p, C.c_size_t, _fp]
        L.mo_generate_serve.argtypes = [C.POINTER(MoModel), C.c_int, C.c_int, _i64p, _szp,
                                        C.c_size_t, C.c_size_t, C.c_int64, _i64p, C.c_size_t, _szp, _fp]
        L.mo_argmax.restype = C.c_size_t
        L.mo_argmax.argtypes = [_fp, C.c_size_t]

    # -- primitives --
    def sumsq(self, x):
        x = f32(x)
        return self.lib.mo_sumsq(_p(x, _fp), x.size)

    def hsum8(self, a):
        a = f32(a)
        return self.lib.mo_hsum8(_p(a, _fp))

    def rstd(self, ss, n, eps):
        return self.lib.mo_rstd(ss, n, eps)

    def _ew(self, name, x):
        x = f32(x)
        out = np.empty_like(x)
        getattr(self.lib, name)(_p(out, _fp), _p(x, _fp), x.size)
        return out

    def sigmoid(self, x):
        return self._ew("mo_sigmoid", x)

    def silu(self, x):
        return self._ew("mo_silu", x)

    def swiglu(self, a, b):
        a, b = f32(a), f32(b)
        out = np.empty_like(a)
        self.lib.mo_swiglu(_p(out, _fp), _p(a, _fp), _p(b, _fp), a.size)
        return out

    def quant_q510(self, y, frac_bits=10):
        y = f32(y)
        q = np.empty(y.shape, np.int32)
        self.lib.mo_quant_q510(_p(q, _i32p), _p(y, _fp), float(1 << frac_bits), y.size)
        return q

    def rmsnorm(self, x, w, eps):
        x, w = f32(x), f32(w)
        rows, cols = x.shape
        y = np.empty_like(x)
        self.lib.mo_rmsnorm(_p(y, _fp), _p(x, _fp), _p(w, _fp), rows, cols, eps)
        return y

    def rmsnorm_swishgate(self, g, o, w, eps):
        g, o, w = f32(g), f32(o), f32(w)
        rows, cols = g.shape
        out = np.empty_like(g)
        self.lib.mo_rmsnorm_swishgate(_p(out, _fp), _p(g, _fp), _p(o, _fp), _p(w, _fp), rows, cols, eps)
        return out

    def hgrn_scan(self, i, f, state=None):
        i, f = f32(i), f32(f)
        T, D = i.shape
        out = np.empty_like(i)
        st = None if state is None else f32(state).copy()
        self.lib.mo_hgrn_scan(_p(out, _fp), _p(i, _fp), _p(f, _fp), T, D, _p(st, _fp))
        return out, st

    def bitlinear(self, x, normw, wq, scale_w, eps, mode, frac_bits=10):
        """Returns dict(out, norm, acc, codes, scale_a) (acc/codes/scale_a for int modes)."""
        x, normw = f32(x), f32(normw)
        wq = np.ascontiguousarray(wq, dtype=np.int8)
        rows, K = x.shape
        N = wq.shape[0]
        out = np.empty((rows, N), np.float32)
        norm = np.empty((rows, K), np.float32)
        acc = np.zeros((rows, N), np.int32)
        codes = np.zeros((rows, K), np.int32)
        sa = np.zeros(rows, np.float32)
        self.lib.mo_bitlinear(_p(out, _fp), _p(x, _fp), _p(normw, _fp), _p(wq, _i8p), scale_w, rows,
                              K, N, eps, mode, frac_bits, _p(norm, _fp), _p(acc, _i32p),
                              _p(codes, _i32p), _p(sa, _fp))
        return dict(out=out, norm=norm, acc=acc, codes=codes, scale_a=sa)

    def ternary_matmul(self, x, wq):
        x = np.ascontiguousarray(x, dtype=np.int32)
        wq = np.ascontiguousarray(wq, dtype=np.int8)
        b, N = x.shape
        M = wq.shape[0]
        acc = np.empty((b, M), np.int32)
        self.lib.mo_ternary_matmul(_p(x, _i32p), _p(acc, _i32p), _p(wq, _i8p), N, M, b)
        return acc

    def argmax(self, v):
        v = f32(v)
        return int(self.lib.mo_argmax(_p(v, _fp), v.size))

    # -- model --
    def model(self, blob):
        return OracleModel(self, blob)


class OracleModel:
    """A blob's tensors viewed as the restatement's mo_model (keeps the views alive)."""

    def __init__(self, oracle: Oracle, blob):
        self.o = oracle
        self.blob = blob
        c = blob.config
        self.cfg = c
        keep = []

        def fp(name):
            a = np.ascontiguousarray(blob.get(name), dtype=np.float32)
            keep.append(a)
            return _p(a, _fp)

        def i8(name):
            a = np.ascontiguousarray(blob.get(name), dtype=np.int8)
            keep.append(a)
            return _p(a, _i8p)

        L = c.num_hidden_layers
        layers = (MoLayer * L)()
        for l in range(L):
            p = f"model.layers.{l}"
            ly = layers[l]
            ly.attn_norm, ly.mlp_norm, ly.g_norm = fp(p + ".attn_norm.w"), fp(p + ".mlp_norm.w"), fp(p + ".g_norm.w")
            for j, tag in enumerate(("i_proj", "f_proj", "g_proj", "o_proj", "gate_proj", "down_proj")):
                ly.wq[j] = i8(f"{p}.{tag}.wq")
                ly.scale_w[j] = float(blob.get(f"{p}.{tag}.scale_w")[0])
                ly.normw[j] = fp(f"{p}.{tag}.normw")
        m = MoModel()
        m.V, m.H, m.L, m.I = c.vocab_size, c.hidden_size, L, c.intermediate_size
        m.eps = c.rms_norm_eps
        m.use_lower_bound = int(c.use_lower_bound)
        m.emb, m.norm_w = fp("model.embeddings"), fp("model.norm.w")
        m.lm_wq, m.lm_scale_w, m.lm_normw = i8("lm_head.wq"), float(blob.get("lm_head.scale_w")[0]), fp("lm_head.normw")
        m.lower_bounds = fp("lower_bounds") if "lower_bounds" in blob.tensors else None
        m.layers = layers
        self.m, self.layers, self.keep = m, layers, keep

    def generate(self, ids, new_tokens, mode=FLOAT, frac_bits=10, eos_id=-1, want_state=False,
                 want_logits=False):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        c = self.cfg
        out = np.empty(ids.size + max(new_tokens, 1), np.int64)
        st = np.empty((c.num_hidden_layers, c.hidden_size), np.float32) if want_state else None
        lg = np.empty(c.vocab_size, np.float32) if want_logits else None
        n = self.o.lib.mo_generate(C.byref(self.m), mode, frac_bits, _p(ids, _i64p), ids.size,
                                   new_tokens, eos_id, _p(out, _i64p), _p(st, _fp), _p(lg, _fp))
        res = [out[:n].copy()]
        if want_state:
            res.append(st)
        if want_logits:
            res.append(lg)
        return res[0] if len(res) == 1 else tuple(res)

    def forward(self, ids, mode=FLOAT, frac_bits=10):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        lg = np.empty((ids.size, self.cfg.vocab_size), np.float32)
        self.o.lib.mo_forward(C.byref(self.m), mode, frac_bits, _p(ids, _i64p), ids.size, _p(lg, _fp))
        return lg

    def generate_serve(self, prompts, new_tokens, mode=FLOAT, frac_bits=10, eos_id=-1, want_state=False):
        """Id stream per stream; with want_state also the final recurrent state [L, B, H]."""
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int64) for p in prompts]))
        lens = np.array([len(p) for p in prompts], np.uintp)
        B = len(prompts)
        cap = int(lens.max()) + max(new_tokens, 1)
        out = np.zeros((B, cap), np.int64)
        out_len = np.zeros(B, np.uintp)
        c = self.cfg
        st = np.empty((c.num_hidden_layers, B, c.hidden_size), np.float32) if want_state else None
        self.o.lib.mo_generate_serve(C.byref(self.m), mode, frac_bits, _p(flat, _i64p),
                                     _p(lens, _szp), B, new_tokens, eos_id, _p(out, _i64p), cap,
                                     _p(out_len, _szp), _p(st, _fp))
        streams = [out[b, :int(out_len[b])].copy() for b in range(B)]
        return (streams, st) if want_state else streams

    def trace(self, ids, mode=FLOAT, frac_bits=10):
        """Stateful prefill layer by layer: (h [L,T,H], state [L,H], internals [L,5,T,H])."""
        c = self.cfg
        ids = np.asarray(ids, np.int64)
        T, H, L = ids.size, c.hidden_size, c.num_hidden_layers
        emb = np.asarray(self.blob.get("model.embeddings"))
        h = np.ascontiguousarray(emb[ids], dtype=np.float32)
        st = np.zeros((L, H), np.float32)
        hs = np.empty((L, T, H), np.float32)
        tr = np.empty((L, 5, T, H), np.float32)
        for l in range(L):
            s = np.ascontiguousarray(st[l])
            trl = np.empty((5, T, H), np.float32)
            self.o.lib.mo_block(C.byref(self.m), mode, frac_bits, _p(h, _fp), T, l, _p(s, _fp), 0,
                                _p(trl, _fp))
            st[l] = s
            hs[l] = h
            tr[l] = trl
        return hs, st, tr


class Ref:
    """The reference engine compiled from its own sources (oracle/_ref)."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (run `make -C oracle ref`)")
        L = self.lib = C.CDLL(path)
        L.ref_last_error.restype = C.c_char_p
        L.ref_sumsq.restype = C.c_float
        L.ref_sumsq.argtypes = [_fp, C.c_size_t]
        L.ref_expf_poly.restype = C.c_float
        L.ref_expf_poly.argtypes = [C.c_float]
        for n in ("ref_sigmoid", "ref_silu"):
            getattr(L, n).argtypes = [_fp, _fp, C.c_size_t]
        L.ref_swiglu_simd.argtypes = [_fp, _fp, _fp, C.c_size_t]
        L.ref_swiglu.argtypes = [_fp, _fp, _fp, C.c_size_t]
        L.ref_quant_q510.argtypes = [_i32p, _fp, C.c_float, C.c_size_t]
        L.ref_ternary_dot_f32.restype = C.c_float
        L.ref_ternary_dot_f32.argtypes = [_fp, _i8p, C.c_size_t]
        L.ref_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_size_t, C.c_size_t, C.c_float]
        L.ref_bitlinear.argtypes = [_fp, _fp, _fp, _i8p, C.c_float, C.c_size_t, C.c_size_t,
                                    C.c_size_t, C.c_float, _fp, C.c_int, C.c_int]
        L.ref_bitlinear_cluster.argtypes = [C.POINTER(_fp), _fp, C.POINTER(_fp), C.POINTER(_i8p),
                                            _fp, C.c_int, C.c_size_t, C.c_size_t, C.c_size_t,
                                            C.c_float, C.c_int]
        L.ref_ternary_matmul.argtypes = [_i32p, _i32p, _i8p, C.c_size_t, C.c_size_t, C.c_size_t]
        L.ref_hgrn_scan.argtypes = [_fp, _fp, _fp, C.c_size_t, C.c_size_t, _fp]
        L.ref_rmsnorm_swishgate.argtypes = [_fp, _fp, _fp, _fp, C.c_size_t, C.c_size_t, C.c_float]
        L.ref_model_open.restype = C.c_void_p
        L.ref_model_open.argtypes = [C.c_char_p, C.c_int, C.c_int]
        L.ref_model_close.argtypes = [C.c_void_p]
        L.ref_model_generate.restype = C.c_long
        L.ref_model_generate.argtypes = [C.c_void_p, _i64p, C.c_size_t, C.c_size_t, C.c_int64,
                                         C.c_float, C.c_int, C.c_uint64, _i64p, C.c_size_t]
        L.ref_model_state.argtypes = [C.c_void_p, _fp]
        L.ref_model_forward.argtypes = [C.c_void_p, _i64p, C.c_size_t, _fp]
        L.ref_model_generate_serve.argtypes = [C.c_void_p, _i64p, _szp, C.c_size_t, C.c_size_t,
                                               C.c_int64, C.c_float, C.c_int, C.c_uint64, _i64p,
                                               C.c_size_t, _szp]
        L.ref_model_trace.argtypes = [C.c_void_p, _i64p, C.c_size_t, _fp, _fp, _fp, _fp, _fp, _fp, _fp]

    def sumsq(self, x):
        x = f32(x)
        return self.lib.ref_sumsq(_p(x, _fp), x.size)

    def _ew(self, name, x):
        x = f32(x)
        out = np.empty_like(x)
        getattr(self.lib, name)(_p(out, _fp), _p(x, _fp), x.size)
        return out

    def sigmoid(self, x):
        return self._ew("ref_sigmoid", x)

    def silu(self, x):
        return self._ew("ref_silu", x)

    def swiglu(self, a, b, chunked=True):
        a, b = f32(a), f32(b)
        out = np.empty_like(a)
        (self.lib.ref_swiglu if chunked else self.lib.ref_swiglu_simd)(
            _p(out, _fp), _p(a, _fp), _p(b, _fp), a.size)
        return out

    def quant_q510(self, y, frac_bits=10):
        y = f32(y)
        q = np.empty(y.shape, np.int32)
        self.lib.ref_quant_q510(_p(q, _i32p), _p(y, _fp), float(1 << frac_bits), y.size)
        return q

    def ternary_dot_f32(self, y, w):
        y = f32(y)
        w = np.ascontiguousarray(w, np.int8)
        return self.lib.ref_ternary_dot_f32(_p(y, _fp), _p(w, _i8p), y.size)

    def rmsnorm(self, x, w, eps):
        x, w = f32(x), f32(w)
        y = np.empty_like(x)
        self.lib.ref_rmsnorm(_p(y, _fp), _p(x, _fp), _p(w, _fp), x.shape[0], x.shape[1], eps)
        return y

    def rmsnorm_swishgate(self, g, o, w, eps):
        g, o, w = f32(g), f32(o), f32(w)
        out = np.empty_like(g)
        self.lib.ref_rmsnorm_swishgate(_p(out, _fp), _p(g, _fp), _p(o, _fp), _p(w, _fp),
                                       g.shape[0], g.shape[1], eps)
        return out

    def hgrn_scan(self, i, f, state=None):
        i, f = f32(i), f32(f)
        out = np.empty_like(i)
        st = None if state is None else f32(state).copy()
        self.lib.ref_hgrn_scan(_p(out, _fp), _p(i, _fp), _p(f, _fp), i.shape[0], i.shape[1], _p(st, _fp))
        return out, st

    def bitlinear(self, x, normw, wq, scale_w, eps, mode, frac_bits=10):
        x, normw = f32(x), f32(normw)
        wq = np.ascontiguousarray(wq, np.int8)
        rows, K = x.shape
        N = wq.shape[0]
        out = np.empty((rows, N), np.float32)
        norm = np.empty((rows, K), np.float32)
        self.lib.ref_bitlinear(_p(out, _fp), _p(x, _fp), _p(normw, _fp), _p(wq, _i8p), scale_w, rows,
                               K, N, eps, _p(norm, _fp), mode, frac_bits)
        return dict(out=out, norm=norm)

    def bitlinear_cluster(self, x, normws, wqs, scales, eps, frac_bits=10):
        x = f32(x)
        rows, K = x.shape
        k = len(wqs)
        N = wqs[0].shape[0]
        outs = [np.empty((rows, N), np.float32) for _ in range(k)]
        nws = [f32(n) for n in normws]
        ws = [np.ascontiguousarray(w, np.int8) for w in wqs]
        sc = f32(scales)
        self.lib.ref_bitlinear_cluster((_fp * k)(*[_p(o, _fp) for o in outs]), _p(x, _fp),
                                       (_fp * k)(*[_p(n, _fp) for n in nws]),
                                       (_i8p * k)(*[_p(w, _i8p) for w in ws]), _p(sc, _fp), k, rows,
                                       K, N, eps, frac_bits)
        return outs

    def ternary_matmul(self, x, wq):
        x = np.ascontiguousarray(x, np.int32)
        wq = np.ascontiguousarray(wq, np.int8)
        b, N = x.shape
        acc = np.empty((b, wq.shape[0]), np.int32)
        self.lib.ref_ternary_matmul(_p(x, _i32p), _p(acc, _i32p), _p(wq, _i8p), N, wq.shape[0], b)
        return acc

    def model(self, blob_path, mode=FLOAT, frac_bits=10):
        return RefModel(self, blob_path, mode, frac_bits)


class RefModel:
    def __init__(self, ref: Ref, blob_path: str, mode: int, frac_bits: int):
        if mode not in (FLOAT, FIXED):
            raise ValueError("the reference engine has Float and FixedQ510 modes only")
        self.r = ref
        self.h = ref.lib.ref_model_open(blob_path.encode(), mode, frac_bits)
        if not self.h:
            raise RuntimeError(ref.lib.ref_last_error().decode())
        from matmulfreellmcpu_amd.blob import read_blob
        self.cfg = read_blob(blob_path).config

    def close(self):
        if self.h:
            self.r.lib.ref_model_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def generate(self, ids, new_tokens, eos_id=-1, temperature=0.0, top_k=0, seed=0):
        ids = np.ascontiguousarray(ids, np.int64)
        cap = ids.size + max(new_tokens, 1)
        out = np.empty(cap, np.int64)
        n = self.r.lib.ref_model_generate(self.h, _p(ids, _i64p), ids.size, new_tokens, eos_id,
                                          temperature, top_k, seed, _p(out, _i64p), cap)
        return out[:n].copy()

    def state(self):
        c = self.cfg
        st = np.empty((c.num_hidden_layers, c.hidden_size), np.float32)
        self.r.lib.ref_model_state(self.h, _p(st, _fp))
        return st

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, np.int64)
        lg = np.empty((ids.size, self.cfg.vocab_size), np.float32)
        self.r.lib.ref_model_forward(self.h, _p(ids, _i64p), ids.size, _p(lg, _fp))
        return lg

    def generate_serve(self, prompts, new_tokens, eos_id=-1, temperature=0.0, top_k=0, seed=0):
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int64) for p in prompts]))
        lens = np.array([len(p) for p in prompts], np.uintp)
        B = len(prompts)
        cap = int(lens.max()) + max(new_tokens, 1)
        out = np.zeros((B, cap), np.int64)
        out_len = np.zeros(B, np.uintp)
        self.r.lib.ref_model_generate_serve(self.h, _p(flat, _i64p), _p(lens, _szp), B, new_tokens,
                                            eos_id, temperature, top_k, seed, _p(out, _i64p), cap,
                                            _p(out_len, _szp))
        return [out[b, :int(out_len[b])].copy() for b in range(B)]

    def trace(self, ids):
        c = self.cfg
        ids = np.ascontiguousarray(ids, np.int64)
        T, H, L = ids.size, c.hidden_size, c.num_hidden_layers
        hs = np.empty((L, T, H), np.float32)
        st = np.empty((L, H), np.float32)
        parts = [np.empty((L, T, H), np.float32) for _ in range(5)]
        self.r.lib.ref_model_trace(self.h, _p(ids, _i64p), T, _p(hs, _fp), _p(st, _fp),
                                   *[_p(p, _fp) for p in parts])
        return hs, st, np.stack(parts, axis=1)
