"""MI355X (gfx950) HGRN-Bit engine: Python binding of the C ABI in include/mmfree_hip.h.

The engine itself is libmmfree_hip.so (HIP kernels + C ABI) with the C++17 ``mmfree`` API
above it; this module is the ctypes plumbing that the tests and bench.py use. There is no
fallback: if the library is not built, or no gfx950 device is present, ``Engine()`` raises.

Device buffers for the operator entry points are raw device addresses (ints: the tests
and bench.py allocate them with the library's own ``mmf_malloc`` and fill them with
``mmf_upload``) or any object with a ``data_ptr()`` method on the same device. Nothing here
imports torch: torch's bundled HIP runtime cannot open a device that this library's runtime
already holds in the same process.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from .blob import Blob, Config, read_blob, LAYER_PROJS  # noqa: F401

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "libmmfree_hip.so")
MKBLOB = os.path.join(HERE, "_lib", "mmfree-mkblob")

FLOAT, FIXED_Q510, INT8_ABSMAX = 0, 1, 2
MODES = {"float": FLOAT, "fixed": FIXED_Q510, "int8": INT8_ABSMAX}

_vp = C.c_void_p
_sz = C.c_size_t
_i64p = C.POINTER(C.c_int64)
_fp = C.POINTER(C.c_float)


class MmfConfig(C.Structure):
    _fields_ = [("vocab_size", _sz), ("hidden_size", _sz), ("num_hidden_layers", _sz),
                ("intermediate_size", _sz), ("use_lower_bound", C.c_int), ("rms_norm_eps", C.c_float)]


TOKEN_CB = C.CFUNCTYPE(None, _vp, C.c_int64)

_lib = None


def load_library(path: str = LIB_PATH):
    """Load libmmfree_hip.so (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
    L = C.CDLL(path)
    i = C.c_int
    sig = {
        "mmf_create": (i, [C.POINTER(_vp), i]),
        "mmf_destroy": (None, [_vp]),
        "mmf_last_error": (C.c_char_p, [_vp]),
        "mmf_sync": (i, [_vp]),
        "mmf_stream": (_vp, [_vp]),
        "mmf_device_info": (i, [_vp, C.c_char_p, _sz, C.POINTER(i)]),
        "mmf_malloc": (i, [_vp, C.POINTER(_vp), _sz]),
        "mmf_free": (i, [_vp, _vp]),
        "mmf_upload": (i, [_vp, _vp, _vp, _sz]),
        "mmf_download": (i, [_vp, _vp, _vp, _sz]),
        "mmf_proj_register": (i, [_vp, _vp, _sz, _sz, C.c_float, _vp, C.POINTER(i)]),
        "mmf_proj_shape": (i, [_vp, i, C.POINTER(_sz), C.POINTER(_sz)]),
        "mmf_ternary_matmul": (i, [_vp, i, _vp, _vp, _sz]),
        "mmf_ternary_matmul_host": (i, [_vp, i, C.POINTER(i), C.POINTER(_vp), C.POINTER(_vp), _sz]),
        "mmf_proj_release": (i, [_vp, i]),
        "mmf_workspace_bytes": (i, [_vp, C.POINTER(_sz)]),
        "mmf_bitlinear": (i, [_vp, i, i, i, C.c_float, _vp, _vp, _sz, _vp]),
        "mmf_bitlinear_noalloc": (i, [_vp, i, i, i, C.c_float, _vp, _vp, _sz, _vp]),
        "mmf_bitlinear_cluster": (i, [_vp, C.POINTER(i), i, i, i, C.c_float, _vp, C.POINTER(_vp), _sz]),
        "mmf_rmsnorm": (i, [_vp, _vp, _vp, _vp, _sz, _sz, C.c_float]),
        "mmf_swiglu": (i, [_vp, _vp, _vp, _vp, _sz]),
        "mmf_hgrn_scan": (i, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
        "mmf_rmsnorm_swishgate": (i, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, C.c_float]),
        "mmf_model_begin": (i, [_vp, C.POINTER(MmfConfig)]),
        "mmf_model_tensor": (i, [_vp, C.c_char_p, i, C.POINTER(_sz), i, _vp]),
        "mmf_model_finalize": (i, [_vp, i, i]),
        "mmf_model_config": (i, [_vp, C.POINTER(MmfConfig)]),
        "mmf_model_generate": (i, [_vp, _i64p, _sz, _sz, C.c_int64, _i64p, _sz, C.POINTER(_sz), TOKEN_CB, _vp]),
        "mmf_model_reset": (i, [_vp, _sz]),
        "mmf_model_prefill": (i, [_vp, _sz, _i64p, _sz, _fp, _i64p]),
        "mmf_model_prefill_streams": (i, [_vp, _sz, _i64p, C.POINTER(C.c_size_t), _fp, _i64p]),
        "mmf_model_step": (i, [_vp, _i64p, _fp, _i64p]),
        "mmf_model_state": (i, [_vp, _fp]),
        "mmf_model_set_scan": (i, [_vp, i]),
        "mmf_model_time_step": (i, [_vp, _i64p, i, i, C.POINTER(C.c_double)]),
        "mmf_model_forward": (i, [_vp, _i64p, _sz, _fp]),
        "mmf_model_trace": (i, [_vp, _i64p, _sz, _fp, _fp, _fp]),
        "mmf_model_time_decode": (i, [_vp, i, i, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "mmf_model_time_prefill": (i, [_vp, _i64p, _sz, i, i, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "mmf_time_bitlinear": (i, [_vp, i, i, i, C.c_float, _vp, _vp, _sz, i, i, C.POINTER(C.c_double),
                                   C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "mmf_measure_peaks": (i, [_vp, C.POINTER(C.c_double)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


class MmfError(RuntimeError):
    pass


def _ptr(x):
    """Device address of an int, or of an object with data_ptr(), or None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _np(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data_as(C.c_void_p)


class Engine:
    """One engine context on one GPU (mmf_create)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = _vp()
        rc = self.lib.mmf_create(C.byref(h), device)
        if rc != 0:
            raise MmfError(f"mmf_create failed ({rc}): {self.lib.mmf_last_error(None).decode()}")
        self.h = h
        self.cfg = None
        self._cb = None

    def close(self):
        if getattr(self, "h", None):
            self.lib.mmf_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _chk(self, rc):
        if rc != 0:
            raise MmfError(f"mmf error {rc}: {self.lib.mmf_last_error(self.h).decode()}")

    def sync(self):
        self._chk(self.lib.mmf_sync(self.h))

    @property
    def stream(self) -> int:
        return self.lib.mmf_stream(self.h) or 0

    def device_info(self):
        buf = C.create_string_buffer(256)
        cus = C.c_int()
        self._chk(self.lib.mmf_device_info(self.h, buf, 256, C.byref(cus)))
        return buf.value.decode(), cus.value

    # ---- projections / operators ----
    def register_proj(self, wq, scale_w: float, normw=None) -> int:
        wq, wp = _np(wq, np.int8)
        nw = None
        if normw is not None:
            nwa, nw = _np(normw, np.float32)
        pid = C.c_int()
        self._chk(self.lib.mmf_proj_register(self.h, wp, wq.shape[0], wq.shape[1], float(scale_w), nw,
                                             C.byref(pid)))
        return pid.value

    def proj_shape(self, pid):
        n, k = _sz(), _sz()
        self._chk(self.lib.mmf_proj_shape(self.h, pid, C.byref(n), C.byref(k)))
        return n.value, k.value

    def bitlinear(self, pid, x, out, rows, mode=FLOAT, frac_bits=10, eps=1e-6, acc=None):
        self._chk(self.lib.mmf_bitlinear(self.h, pid, mode, frac_bits, eps, _ptr(x), _ptr(out), rows, _ptr(acc)))

    def bitlinear_noalloc(self, pid, x, out, rows, mode=FLOAT, frac_bits=10, eps=1e-6, acc=None):
        """mmf_bitlinear with its scratch in the library's static device array (no allocation)."""
        self._chk(self.lib.mmf_bitlinear_noalloc(self.h, pid, mode, frac_bits, eps, _ptr(x), _ptr(out), rows,
                                                 _ptr(acc)))

    def bitlinear_cluster(self, pids, x, outs, rows, mode=FLOAT, frac_bits=10, eps=1e-6):
        k = len(pids)
        ids = (C.c_int * k)(*pids)
        op = (_vp * k)(*[_ptr(o) for o in outs])
        self._chk(self.lib.mmf_bitlinear_cluster(self.h, ids, k, mode, frac_bits, eps, _ptr(x), op, rows))

    def ternary_matmul(self, pid, x, acc, b):
        self._chk(self.lib.mmf_ternary_matmul(self.h, pid, _ptr(x), _ptr(acc), b))

    def ternary_matmul_host(self, pids, xs):
        """k projections on host arrays in one round trip: xs[z] int32 [b, K_z] -> int32 [b, N_z]."""
        k = len(pids)
        b = xs[0].shape[0]
        xs = [np.ascontiguousarray(x, np.int32) for x in xs]
        accs = [np.zeros((b, self.proj_shape(p)[0]), np.int32) for p in pids]
        ids = (C.c_int * k)(*pids)
        xp = (_vp * k)(*[x.ctypes.data for x in xs])
        ap = (_vp * k)(*[a.ctypes.data for a in accs])
        self._chk(self.lib.mmf_ternary_matmul_host(self.h, k, ids, xp, ap, b))
        return accs

    def proj_release(self, pid):
        self._chk(self.lib.mmf_proj_release(self.h, pid))

    def workspace_bytes(self):
        n = _sz()
        self._chk(self.lib.mmf_workspace_bytes(self.h, C.byref(n)))
        return n.value

    def rmsnorm(self, y, x, w, rows, cols, eps=1e-6):
        self._chk(self.lib.mmf_rmsnorm(self.h, _ptr(y), _ptr(x), _ptr(w), rows, cols, eps))

    def swiglu(self, out, a, b, n):
        self._chk(self.lib.mmf_swiglu(self.h, _ptr(out), _ptr(a), _ptr(b), n))

    def hgrn_scan(self, out, i, f, T, D, state=None):
        self._chk(self.lib.mmf_hgrn_scan(self.h, _ptr(out), _ptr(i), _ptr(f), T, D, _ptr(state)))

    def rmsnorm_swishgate(self, out, g, o, w, rows, cols, eps=1e-6):
        self._chk(self.lib.mmf_rmsnorm_swishgate(self.h, _ptr(out), _ptr(g), _ptr(o), _ptr(w), rows, cols, eps))

    # ---- model ----
    def load_blob(self, path_or_blob, mode=FLOAT, frac_bits=10):
        """Upload every tensor of an MMFREE1 blob and prepare the engine for `mode`."""
        blob = read_blob(path_or_blob) if isinstance(path_or_blob, str) else path_or_blob
        c = blob.config
        cfg = MmfConfig(c.vocab_size, c.hidden_size, c.num_hidden_layers, c.intermediate_size,
                        int(c.use_lower_bound), c.rms_norm_eps)
        self._chk(self.lib.mmf_model_begin(self.h, C.byref(cfg)))
        for name, arr in blob.tensors.items():
            a = np.ascontiguousarray(arr)
            shape = (_sz * max(a.ndim, 1))(*a.shape)
            dt = 1 if a.dtype == np.int8 else 0
            self._chk(self.lib.mmf_model_tensor(self.h, name.encode(), dt, shape, a.ndim,
                                                a.ctypes.data_as(_vp)))
        self._chk(self.lib.mmf_model_finalize(self.h, mode, frac_bits))
        self.cfg = c
        self.mode = mode
        return self

    def generate(self, ids, new_tokens, eos_id=-1, on_token=None):
        ids, ip = _np(ids, np.int64)
        cap = ids.size + new_tokens
        out = np.zeros(max(cap, 1), np.int64)
        n = _sz()
        cb = TOKEN_CB(lambda _u, t: on_token(int(t))) if on_token else TOKEN_CB()
        self._cb = cb
        self._chk(self.lib.mmf_model_generate(self.h, ids.ctypes.data_as(_i64p), ids.size, new_tokens, eos_id,
                                              out.ctypes.data_as(_i64p), cap, C.byref(n), cb, None))
        return out[:n.value].copy()

    def reset(self, streams=1):
        self._chk(self.lib.mmf_model_reset(self.h, streams))
        self.streams = streams

    def prefill(self, stream, ids, want_logits=False):
        ids = np.ascontiguousarray(ids, np.int64)
        lg = np.empty(self.cfg.vocab_size, np.float32) if want_logits else None
        am = np.zeros(1, np.int64)
        self._chk(self.lib.mmf_model_prefill(self.h, stream, ids.ctypes.data_as(_i64p), ids.size,
                                             lg.ctypes.data_as(_fp) if lg is not None else None,
                                             am.ctypes.data_as(_i64p)))
        return (int(am[0]), lg) if want_logits else int(am[0])

    def prefill_streams(self, prompts, want_logits=False):
        """Prefill streams 0..len(prompts)-1 together (mmf_model_prefill_streams): the same
        first tokens, logits and states as one prefill() per stream in order."""
        ids = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int64).ravel() for p in prompts]), np.int64)
        lens = np.ascontiguousarray([len(p) for p in prompts], np.uint64)
        n = lens.size
        lg = np.empty((n, self.cfg.vocab_size), np.float32) if want_logits else None
        am = np.zeros(n, np.int64)
        self._chk(self.lib.mmf_model_prefill_streams(self.h, n, ids.ctypes.data_as(_i64p),
                                                     lens.ctypes.data_as(C.POINTER(C.c_size_t)),
                                                     lg.ctypes.data_as(_fp) if lg is not None else None,
                                                     am.ctypes.data_as(_i64p)))
        return (am, lg) if want_logits else am

    def step(self, tokens, want_logits=False):
        t = np.ascontiguousarray(tokens, np.int64)
        B = t.size
        lg = np.empty((B, self.cfg.vocab_size), np.float32) if want_logits else None
        am = np.zeros(B, np.int64)
        self._chk(self.lib.mmf_model_step(self.h, t.ctypes.data_as(_i64p),
                                          lg.ctypes.data_as(_fp) if lg is not None else None,
                                          am.ctypes.data_as(_i64p)))
        return (am, lg) if want_logits else am

    def set_scan(self, chunked: bool):
        """Float-mode prefill recurrence: time-ordered (default, bit-exact) or chunked parallel."""
        self._chk(self.lib.mmf_model_set_scan(self.h, 1 if chunked else 0))

    def state(self):
        c = self.cfg
        st = np.empty((c.num_hidden_layers, getattr(self, "streams", 1), c.hidden_size), np.float32)
        self._chk(self.lib.mmf_model_state(self.h, st.ctypes.data_as(_fp)))
        return st

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, np.int64)
        lg = np.empty((ids.size, self.cfg.vocab_size), np.float32)
        self._chk(self.lib.mmf_model_forward(self.h, ids.ctypes.data_as(_i64p), ids.size, lg.ctypes.data_as(_fp)))
        return lg

    def trace(self, ids, internals=True):
        c = self.cfg
        ids = np.ascontiguousarray(ids, np.int64)
        T, H, L = ids.size, c.hidden_size, c.num_hidden_layers
        h = np.empty((L, T, H), np.float32)
        st = np.empty((L, H), np.float32)
        it = np.empty((L, 5, T, H), np.float32) if internals else None
        self._chk(self.lib.mmf_model_trace(self.h, ids.ctypes.data_as(_i64p), T, h.ctypes.data_as(_fp),
                                           st.ctypes.data_as(_fp), it.ctypes.data_as(_fp) if internals else None))
        self.streams = 1
        return h, st, it

    def time_decode(self, warmup=3, reps=20):
        step = C.c_double()
        kinds = (C.c_double * 5)()
        self._chk(self.lib.mmf_model_time_decode(self.h, warmup, reps, C.byref(step), kinds))
        return step.value, dict(zip(("ifg", "o", "gate", "down", "lm"), list(kinds)))

    PREFILL_KINDS = ("prologue", "gemm_ifg", "mixer", "gemm_o", "gemm_gate", "gemm_down", "lm", "embed")

    def time_prefill(self, ids, warmup=1, reps=3, kinds=True):
        """Microseconds per prefill (prompt through all layers + final norm/lm_head/argmax of
        the last position) and, with kinds, the microseconds per prefill of each launch kind."""
        ids, _ = _np(ids, np.int64)
        total = C.c_double()
        k = (C.c_double * 8)()
        self._chk(self.lib.mmf_model_time_prefill(self.h, ids.ctypes.data_as(_i64p), ids.size, warmup, reps,
                                                  C.byref(total), k if kinds else None))
        return total.value, (dict(zip(self.PREFILL_KINDS, list(k))) if kinds else None)

    def time_step_kinds(self, tokens, warmup=1, reps=4):
        """Microseconds per serving step in each launch kind (launches timed one by one)."""
        tokens, _ = _np(tokens, np.int64)
        k = (C.c_double * 8)()
        self._chk(self.lib.mmf_model_time_step(self.h, tokens.ctypes.data_as(_i64p), warmup, reps, k))
        return dict(zip(self.PREFILL_KINDS, list(k)))

    def measure_peaks(self):
        """Measured device ceilings: HBM and Infinity Cache read GB/s, int8 MFMA TOP/s, fp32
        FMA TFLOP/s (each from a kernel doing only that work)."""
        v = (C.c_double * 4)()
        self._chk(self.lib.mmf_measure_peaks(self.h, v))
        return {"hbm_read_GBps": round(v[0], 1), "mall_read_GBps": round(v[1], 1),
                "int8_mfma_TOPS": round(v[2], 1), "fp32_fma_TFLOPS": round(v[3], 2)}

    def time_bitlinear(self, proj_id, x, out, rows, mode=FLOAT, frac_bits=10, eps=1e-6, warmup=3, reps=20):
        """(total, prologue, gemm) microseconds per mmf_bitlinear call on device buffers."""
        t, p, g = C.c_double(), C.c_double(), C.c_double()
        self._chk(self.lib.mmf_time_bitlinear(self.h, proj_id, mode, frac_bits, eps, _ptr(x), _ptr(out), rows,
                                              warmup, reps, C.byref(t), C.byref(p), C.byref(g)))
        return t.value, p.value, g.value


def make_blob(path: str, preset: str | None = None, seed: int = 1234, vocab=None, hidden=None, layers=None,
              inter=None, random_norms=False, random_lb=False, lower_bound=True) -> str:
    """Write a seeded synthetic MMFREE1 blob with the in-tree mmfree-mkblob tool."""
    import subprocess
    if not os.path.exists(MKBLOB):
        raise RuntimeError(f"{MKBLOB} is not built")
    cmd = [MKBLOB, "--out", path, "--seed", str(seed)]
    if preset:
        cmd += ["--preset", preset]
    for flag, v in (("--vocab", vocab), ("--hidden", hidden), ("--layers", layers), ("--inter", inter)):
        if v is not None:
            cmd += [flag, str(v)]
    if random_norms:
        cmd.append("--random-norms")
    if random_lb:
        cmd.append("--random-lb")
    if not lower_bound:
        cmd.append("--no-lower-bound")
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return path
