"""mmf_bitlinear_noalloc (scratch in the library's static device array) against mmf_bitlinear.

Both entry points run the same kernels; the no-alloc one takes the activation codes and the
split-K partials from one fixed region per GPU that keeps the previous call's contents. So
every case runs two calls in a row, the second on a smaller input than the first, and each
call must equal mmf_bitlinear on the same inputs bit for bit (outputs and int32
accumulators), and the oracle.
"""
import ctypes as C

import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu

FLOAT, FIXED, INT8 = 0, 1, 2


@pytest.fixture(scope="module")
def eng():
    from matmulfreellmcpu_amd import Engine
    e = Engine(0)
    yield e
    e.close()


class Buf:
    def __init__(self, eng, arr=None, shape=None, dtype=np.float32):
        self.eng = eng
        if arr is not None:
            arr = np.ascontiguousarray(arr)
            shape, dtype = arr.shape, arr.dtype
        self.shape, self.dtype = tuple(shape), np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        eng._chk(eng.lib.mmf_malloc(eng.h, C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value
        if arr is not None:
            eng._chk(eng.lib.mmf_upload(eng.h, self.ptr, arr.ctypes.data_as(C.c_void_p), self.nbytes))

    def get(self):
        out = np.empty(self.shape, self.dtype)
        self.eng._chk(self.eng.lib.mmf_download(self.eng.h, out.ctypes.data_as(C.c_void_p), self.ptr, self.nbytes))
        return out

    def free(self):
        if self.ptr:
            self.eng.lib.mmf_free(self.eng.h, self.ptr)
            self.ptr = None


def _case(eng, oracle, rows, K, N, mode, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, K)) * 2).astype(np.float32)
    x[rows // 2] *= 40.0  # saturating Q5.10 codes in one row
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    sw = float(np.float32(1.0 / 0.0163))
    pid = eng.register_proj(wq, sw, nw)
    dx = Buf(eng, x)
    outs = {}
    for name in ("noalloc", "alloc"):
        dout = Buf(eng, shape=(rows, N))
        dacc = Buf(eng, shape=(rows, N), dtype=np.int32) if mode != FLOAT else None
        fn = eng.bitlinear_noalloc if name == "noalloc" else eng.bitlinear
        fn(pid, dx.ptr, dout.ptr, rows, mode=mode, acc=dacc.ptr if dacc else None)
        eng.sync()
        outs[name] = (dout.get(), dacc.get() if dacc else None)
        dout.free()
        if dacc:
            dacc.free()
    dx.free()
    what = f"rows={rows} K={K} N={N} mode={mode}"
    assert_bitexact(outs["noalloc"][0], outs["alloc"][0], "noalloc vs bitlinear out " + what)
    want = oracle.bitlinear(x, nw, wq, sw, 1e-6, mode)
    assert_bitexact(outs["noalloc"][0], want["out"], "noalloc vs oracle out " + what)
    if mode != FLOAT:
        np.testing.assert_array_equal(outs["noalloc"][1], outs["alloc"][1])
        np.testing.assert_array_equal(outs["noalloc"][1], want["acc"])


# (rows, K, N): the first call of each pair is the larger one. 300 rows take the matrix
# cores; 40 rows x K 2048 split K over 8 blocks in the integer modes (partials in the
# scratch); 1 row is the single-row path; K 1031 leaves a 7-element tail.
PAIRS = [((300, 2816, 1024), (40, 2048, 512)), ((40, 2048, 512), (1, 1031, 96)), ((130, 1024, 333), (17, 256, 128))]


@pytest.mark.parametrize("first,second", PAIRS)
@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
def test_noalloc_matches_bitlinear(eng, oracle, first, second, mode):
    print(f"noalloc pair {first} -> {second} mode={mode}", flush=True)
    _case(eng, oracle, *first, mode, seed=sum(first) + mode)
    _case(eng, oracle, *second, mode, seed=sum(second) + 7 * mode)


@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
def test_noalloc_allocates_nothing(oracle, mode):
    """On a fresh context the no-alloc entry point leaves the context's grow-only workspace
    empty (the activation codes and split-K partials live in the static scratch), while one
    mmf_bitlinear call of the same shape allocates it: the query sees allocations."""
    from matmulfreellmcpu_amd import Engine
    e = Engine(0)
    try:
        rows, K, N = 40, 2048, 512  # the integer modes split K here: partials in the scratch too
        rng = np.random.default_rng(31 + mode)
        x = rng.standard_normal((rows, K)).astype(np.float32)
        nw = np.ones(K, np.float32)
        wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
        pid = e.register_proj(wq, 25.0, nw)
        dx, dout = Buf(e, x), Buf(e, shape=(rows, N))
        assert e.workspace_bytes() == 0
        for _ in range(2):
            e.bitlinear_noalloc(pid, dx.ptr, dout.ptr, rows, mode=mode)
            e.sync()
            assert e.workspace_bytes() == 0, "mmf_bitlinear_noalloc allocated workspace"
        assert_bitexact(dout.get(), oracle.bitlinear(x, nw, wq, 25.0, 1e-6, mode)["out"], "noalloc on a fresh context")
        e.bitlinear(pid, dx.ptr, dout.ptr, rows, mode=mode)
        e.sync()
        assert e.workspace_bytes() > 0
        dx.free()
        dout.free()
    finally:
        e.close()


def test_noalloc_refuses_oversize(eng):
    """A call needing more than the static scratch fails before any launch, with a message."""
    from matmulfreellmcpu_amd import MmfError
    rows, K, N = 4096, 5632, 64  # float activations: 4096 x 5640 x 4 bytes > 64 MiB
    rng = np.random.default_rng(5)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    pid = eng.register_proj(wq, 30.0, np.ones(K, np.float32))
    dx, dout = Buf(eng, shape=(rows, K)), Buf(eng, shape=(rows, N))
    with pytest.raises(MmfError, match="static scratch"):
        eng.bitlinear_noalloc(pid, dx.ptr, dout.ptr, rows, mode=FLOAT)
    dx.free()
    dout.free()
