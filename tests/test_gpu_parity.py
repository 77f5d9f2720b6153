"""Parity of the HIP path (through the C ABI) with the CPU restatement of the reference.

Bar: bit-exact everywhere -- integer accumulators and codes, and fp32 outputs of the Float
and FixedQ510 modes (the HIP kernels keep the reference's summation order and FMA sites).
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
    print("device:", e.device_info(), flush=True)
    yield e
    e.close()


class Dev:
    """Device buffer from the engine's allocator, filled from / read into numpy."""

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

    def __del__(self):
        try:
            self.eng.lib.mmf_free(self.eng.h, self.ptr)
        except Exception:
            pass


SHAPES = [(1, 64, 64), (3, 176, 48), (5, 1024, 333), (1, 1031, 17), (9, 100, 40), (2, 7, 19), (17, 256, 128)]


@pytest.mark.parametrize("rows,K,N", SHAPES)
@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
def test_bitlinear_op(eng, oracle, rows, K, N, mode):
    print(f"bitlinear rows={rows} K={K} N={N} mode={mode}", flush=True)
    rng = np.random.default_rng(rows * 1000 + K + N + mode)
    x = (rng.standard_normal((rows, K)) * 2).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    sw = float(np.float32(1.0 / 0.0157))
    want = oracle.bitlinear(x, nw, wq, sw, 1e-6, mode)
    pid = eng.register_proj(wq, sw, nw)
    dx, dout = Dev(eng, x), Dev(eng, shape=(rows, N))
    dacc = Dev(eng, shape=(rows, N), dtype=np.int32)
    eng.bitlinear(pid, dx.ptr, dout.ptr, rows, mode=mode, acc=dacc.ptr if mode else None)
    eng.sync()
    if mode:
        np.testing.assert_array_equal(dacc.get(), want["acc"])
    assert_bitexact(dout.get(), want["out"], f"bitlinear out mode {mode}")


@pytest.mark.parametrize("rows,K,N", [(64, 1024, 6176), (57, 1024, 6176), (1030, 512, 2048), (1030, 523, 2048)])
@pytest.mark.parametrize("mode", [FIXED, INT8])
def test_bitlinear_op_kgroups(eng, oracle, rows, K, N, mode):
    """K-groups in the matrix-core GEMM: a 64-row tile with 49 column tiles (four groups
    per block) and 128 x 128 tiles at one block per CU (two groups), ragged rows and a K
    tail included; the groups' partial tiles are added in LDS."""
    print(f"bitlinear k-groups rows={rows} K={K} N={N} mode={mode}", flush=True)
    rng = np.random.default_rng(rows * 7 + K + mode)
    x = (rng.standard_normal((rows, K)) * 2).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    sw = float(np.float32(1.0 / 0.0157))
    want = oracle.bitlinear(x, nw, wq, sw, 1e-6, mode)
    pid = eng.register_proj(wq, sw, nw)
    dx, dout = Dev(eng, x), Dev(eng, shape=(rows, N))
    dacc = Dev(eng, shape=(rows, N), dtype=np.int32)
    eng.bitlinear(pid, dx.ptr, dout.ptr, rows, mode=mode, acc=dacc.ptr)
    eng.sync()
    np.testing.assert_array_equal(dacc.get(), want["acc"])
    assert_bitexact(dout.get(), want["out"], f"bitlinear k-groups out mode {mode}")


@pytest.mark.parametrize("rows,K,N", [(16, 64, 64), (64, 1024, 2560), (100, 1031, 333), (1030, 523, 2048),
                                      (1030, 523, 8192), (2048, 256, 4008)])
def test_bitlinear_op_float_mfma(eng, oracle, rows, K, N):
    """Float mode on the fp32 matrix cores, one reference lane chain per wave: 32 x 64 tiles
    of the 32x32 instruction (the last three shapes) and 16 x 64 tiles of the 16x16 one (the
    first three), the chain tiles added in LDS; ragged rows and columns, K tails."""
    print(f"bitlinear float mfma rows={rows} K={K} N={N}", flush=True)
    rng = np.random.default_rng(rows * 3 + K + N)
    x = (rng.standard_normal((rows, K)) * 2).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    sw = float(np.float32(1.0 / 0.0157))
    want = oracle.bitlinear(x, nw, wq, sw, 1e-6, FLOAT)
    pid = eng.register_proj(wq, sw, nw)
    dx, dout = Dev(eng, x), Dev(eng, shape=(rows, N))
    eng.bitlinear(pid, dx.ptr, dout.ptr, rows, mode=FLOAT)
    eng.sync()
    assert_bitexact(dout.get(), want["out"], "bitlinear float mfma")


@pytest.mark.parametrize("rows,K,N", [(64, 1024, 512), (256, 1000, 1600)])
def test_bitlinear_op_float_mfma_denormal(eng, oracle, rows, K, N):
    """The fp32 matrix-core chains through the denormal range: norm weights near 1e-38 make
    the BitLinear inputs and most chain sums denormal, so each matrix op must keep the
    reference's denormal sums and roundings (16 x 64 tiles at 64 rows, 32 x 64 tiles at 256
    rows)."""
    print(f"bitlinear float mfma denormal rows={rows} K={K} N={N}", flush=True)
    rng = np.random.default_rng(rows + K * 7 + N)
    x = (rng.standard_normal((rows, K)) * 2).astype(np.float32)
    nw = (rng.uniform(0.05, 3.0, K) * 1e-38).astype(np.float32)
    nw[::7] *= -1.0
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    sw = float(np.float32(1.0 / 0.0157))
    want = oracle.bitlinear(x, nw, wq, sw, 1e-6, FLOAT)
    tiny = np.abs(want["out"]) < np.float32(1.17549435e-38)
    assert tiny.mean() > 0.5  # most outputs are denormal (the check exercises that range)
    pid = eng.register_proj(wq, sw, nw)
    dx, dout = Dev(eng, x), Dev(eng, shape=(rows, N))
    eng.bitlinear(pid, dx.ptr, dout.ptr, rows, mode=FLOAT)
    eng.sync()
    assert_bitexact(dout.get(), want["out"], "bitlinear float mfma denormal")


def test_measured_ceilings(eng):
    """The calibration kernels run and give rates below the published peaks (HBM 8 TB/s,
    int8 dense 5.0 POP/s, fp32 vector FMA without packing 78.6 TFLOP/s) and well above zero."""
    p = eng.measure_peaks()
    print("ceilings:", p, flush=True)
    assert 1000 < p["hbm_read_GBps"] < 8500
    assert p["mall_read_GBps"] > 1000
    assert 500 < p["int8_mfma_TOPS"] < 5100
    assert 10 < p["fp32_fma_TFLOPS"] < 80


def test_bitlinear_cluster_matches_single(eng, oracle):
    rng = np.random.default_rng(5)
    rows, K, N = 4, 256, 96
    x = rng.standard_normal((rows, K)).astype(np.float32)
    pids, wants = [], []
    for j in range(3):
        nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
        wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
        pids.append(eng.register_proj(wq, 40.0 + j, nw))
        wants.append(oracle.bitlinear(x, nw, wq, 40.0 + j, 1e-6, FIXED)["out"])
    dx = Dev(eng, x)
    outs = [Dev(eng, shape=(rows, N)) for _ in range(3)]
    eng.bitlinear_cluster(pids, dx.ptr, [o.ptr for o in outs], rows, mode=FIXED)
    eng.sync()
    for o, w in zip(outs, wants):
        assert_bitexact(o.get(), w, "cluster")


@pytest.mark.parametrize("b,K,N", [(1, 1024, 256), (4, 2816, 64), (3, 13, 5)])
def test_ternary_matmul(eng, oracle, b, K, N):
    rng = np.random.default_rng(b + K)
    x = rng.integers(-32768, 32768, (b, K)).astype(np.int32)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    pid = eng.register_proj(wq, 1.0)
    dx, dacc = Dev(eng, x), Dev(eng, shape=(b, N), dtype=np.int32)
    eng.ternary_matmul(pid, dx.ptr, dacc.ptr, b)
    eng.sync()
    np.testing.assert_array_equal(dacc.get(), oracle.ternary_matmul(x, wq))


def test_ternary_matmul_host_k_projections(eng, oracle):
    """mmf_ternary_matmul_host: three projections of different shapes on host buffers in one
    round trip (the seam's matmul_seq), against the exact integer product; a released
    projection is refused afterwards and the others keep working."""
    from matmulfreellmcpu_amd import MmfError
    rng = np.random.default_rng(19)
    b = 3
    shapes = [(1024, 256), (2816, 64), (13, 5)]
    ws = [rng.integers(-1, 2, (N, K)).astype(np.int8) for K, N in shapes]
    xs = [rng.integers(-32768, 32768, (b, K)).astype(np.int32) for K, _ in shapes]
    pids = [eng.register_proj(w, 1.0) for w in ws]
    for rep in range(2):  # staging buffers reused on the second call
        accs = eng.ternary_matmul_host(pids, xs)
        for x, w, a in zip(xs, ws, accs):
            np.testing.assert_array_equal(a, oracle.ternary_matmul(x, w))
    # one shape, few rows: the single-kernel path (int32 dot on the resident slab, accumulators
    # written into the pinned staging); K with a tail, N not a multiple of 16
    same = [rng.integers(-1, 2, (77, 1003)).astype(np.int8) for _ in range(3)]
    sp = [eng.register_proj(w, 1.0) for w in same]
    for b1 in (1, 4):
        x1 = [rng.integers(-32768, 32768, (b1, 1003)).astype(np.int32) for _ in range(3)]
        for x, w, a in zip(x1, same, eng.ternary_matmul_host(sp, x1)):
            np.testing.assert_array_equal(a, oracle.ternary_matmul(x, w))
    eng.proj_release(pids[1])
    with pytest.raises(MmfError, match="released"):
        eng.ternary_matmul_host([pids[1]], [xs[1]])
    with pytest.raises(MmfError):
        eng.proj_release(pids[1])
    accs = eng.ternary_matmul_host([pids[2], pids[0]], [xs[2], xs[0]])
    np.testing.assert_array_equal(accs[0], oracle.ternary_matmul(xs[2], ws[2]))
    np.testing.assert_array_equal(accs[1], oracle.ternary_matmul(xs[0], ws[0]))


def test_model_projection_cannot_be_released(blobs):
    from matmulfreellmcpu_amd import FLOAT, Engine, MmfError, read_blob
    e = Engine(0)
    try:
        e.load_blob(read_blob(blobs("tiny")), FLOAT)
        with pytest.raises(MmfError, match="loaded model"):
            e.proj_release(0)
    finally:
        e.close()


def test_elementwise_ops(eng, oracle):
    rng = np.random.default_rng(3)
    for n in (8, 13, 8192 + 5, 20000):
        a = (rng.standard_normal(n) * 8).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        da, db, do = Dev(eng, a), Dev(eng, b), Dev(eng, shape=(n,))
        eng.swiglu(do.ptr, da.ptr, db.ptr, n)
        eng.sync()
        # activations.cpp:9-15 splits into 8192-element SIMD calls
        want = np.concatenate([oracle.swiglu(a[o:o + 8192], b[o:o + 8192]) for o in range(0, n, 8192)])
        assert_bitexact(do.get(), want, f"swiglu n={n}")
    for rows, cols in ((3, 64), (2, 100), (1, 2560)):
        g = rng.standard_normal((rows, cols)).astype(np.float32) * 3
        o = rng.standard_normal((rows, cols)).astype(np.float32) * 3
        w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
        dg, dob, dw, dy = Dev(eng, g), Dev(eng, o), Dev(eng, w), Dev(eng, shape=(rows, cols))
        eng.rmsnorm(dy.ptr, dg.ptr, dw.ptr, rows, cols)
        eng.sync()
        assert_bitexact(dy.get(), oracle.rmsnorm(g, w, 1e-6), "rmsnorm")
        eng.rmsnorm_swishgate(dy.ptr, dg.ptr, dob.ptr, dw.ptr, rows, cols)
        eng.sync()
        assert_bitexact(dy.get(), oracle.rmsnorm_swishgate(g, o, w, 1e-6), "swishgate")
    T, D = 37, 200
    i = rng.standard_normal((T, D)).astype(np.float32)
    f = rng.uniform(0, 1, (T, D)).astype(np.float32)
    st = rng.standard_normal(D).astype(np.float32)
    di, df, dout, dst = Dev(eng, i), Dev(eng, f), Dev(eng, shape=(T, D)), Dev(eng, st)
    eng.hgrn_scan(dout.ptr, di.ptr, df.ptr, T, D, dst.ptr)
    eng.sync()
    wo, wst = oracle.hgrn_scan(i, f, st)
    assert_bitexact(dout.get(), wo, "scan out")
    assert_bitexact(dst.get(), wst, "scan state")


def _model(eng_cls, blob, mode):
    e = eng_cls(0)
    e.load_blob(blob, mode)
    return e


@pytest.mark.parametrize("name", ["tiny", "tiny_nolb", "small", "odd"])
@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
def test_generate_matches_oracle(blobs, oracle, name, mode):
    from matmulfreellmcpu_amd import Engine, read_blob
    print(f"generate blob={name} mode={mode}", flush=True)
    blob = read_blob(blobs(name))
    om = oracle.model(blob)
    rng = np.random.default_rng(42)
    V = blob.config.vocab_size
    ids = rng.integers(3, V, 9)
    want, wst, wlg = om.generate(ids, 24, mode, want_state=True, want_logits=True)
    e = Engine(0)
    e.load_blob(blob, mode)
    got = e.generate(ids, 24)
    np.testing.assert_array_equal(got, want)
    assert_bitexact(e.state()[:, 0, :], wst, "final recurrent state")
    # second call replays the captured decode graph from a fresh state
    np.testing.assert_array_equal(e.generate(ids, 24), want)
    e.close()


@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
def test_trace_per_layer(blobs, oracle, mode):
    from matmulfreellmcpu_amd import Engine, read_blob
    blob = read_blob(blobs("small"))
    om = oracle.model(blob)
    ids = np.arange(5, 5 + 33) * 97 % blob.config.vocab_size
    wh, wst, wtr = om.trace(ids, mode)
    e = Engine(0)
    e.load_blob(blob, mode)
    h, st, tr = e.trace(ids)
    for l in range(blob.config.num_hidden_layers):
        for k, nm in enumerate(("i", "f", "g", "scan", "recur")):
            assert_bitexact(tr[l, k], wtr[l, k], f"layer {l} {nm}")
        assert_bitexact(h[l], wh[l], f"layer {l} h")
        assert_bitexact(st[l], wst[l], f"layer {l} state")
    e.close()


@pytest.mark.parametrize("mode", [FLOAT, FIXED])
def test_forward_logits(blobs, oracle, mode):
    from matmulfreellmcpu_amd import Engine, read_blob
    blob = read_blob(blobs("tiny"))
    om = oracle.model(blob)
    ids = np.array([3, 17, 200, 45, 7, 300, 2, 99, 511, 0, 1])
    e = Engine(0)
    e.load_blob(blob, mode)
    assert_bitexact(e.forward(ids), om.forward(ids, mode), "forward logits")
    e.close()


def test_forward_float_mid_prompt(blobs, oracle):
    """600-token float forward on hidden 1024: every GEMM kind runs on the 32 x 64 tiles of
    the 32x32 matrix-core instruction (store, residual add, swiglu pair, ragged last tile)."""
    from matmulfreellmcpu_amd import Engine, read_blob
    print("forward float mid prompt", flush=True)
    blob = read_blob(blobs("wide"))
    om = oracle.model(blob)
    ids = np.random.default_rng(19).integers(3, blob.config.vocab_size, 600)
    want = om.forward(ids, FLOAT)
    e = Engine(0)
    e.load_blob(blob, FLOAT)
    assert_bitexact(e.forward(ids), want, "mid-prompt forward logits")
    e.close()


def test_forward_float_long_prompt(blobs, oracle):
    """6144-token float forward: every GEMM kind (i/f/g store, o and down residual add, the
    gate/up swiglu pair) runs on the 32 x 64 matrix-core tiles with hidden 768 and a K of
    528 for down_proj; all logits bit for bit."""
    from matmulfreellmcpu_amd import Engine, read_blob
    print("forward float long prompt", flush=True)
    blob = read_blob(blobs("tall"))
    om = oracle.model(blob)
    ids = np.random.default_rng(17).integers(3, blob.config.vocab_size, 6144)
    want = om.forward(ids, FLOAT)
    e = Engine(0)
    e.load_blob(blob, FLOAT)
    assert_bitexact(e.forward(ids), want, "long-prompt forward logits")
    e.close()


@pytest.mark.parametrize("name", ["small", "odd"])
@pytest.mark.parametrize("mode", [FLOAT, FIXED])
def test_serve_matches_oracle(blobs, oracle, name, mode):
    """Serving steps of 5 streams; the recurrence step runs inside the g_norm prologue.
    "odd" (hidden 100): the last 4 of the 5 x 100 mixer elements take the scalar tail."""
    from matmulfreellmcpu_amd import Engine, read_blob
    print(f"serve blob={name} mode={mode}", flush=True)
    blob = read_blob(blobs(name))
    om = oracle.model(blob)
    rng = np.random.default_rng(9)
    V = blob.config.vocab_size
    prompts = [rng.integers(3, V, n) for n in (5, 12, 1, 7, 5)]
    prompts[4] = prompts[0].copy()  # identical prompts must give identical streams
    want = om.generate_serve(prompts, 10, mode)
    e = Engine(0)
    e.load_blob(blob, mode)
    B = len(prompts)
    e.reset(B)
    streams = [list(p) for p in prompts]
    for b in range(B):
        streams[b].append(e.prefill(b, prompts[b]))
    for _ in range(9):
        nxt = e.step([s[-1] for s in streams])
        for b in range(B):
            streams[b].append(int(nxt[b]))
    for b in range(B):
        np.testing.assert_array_equal(np.array(streams[b]), want[b])
    np.testing.assert_array_equal(streams[0], streams[4])
    e.close()


@pytest.mark.parametrize("name", ["small", "odd"])
@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
def test_prefill_streams_matches_per_stream(blobs, name, mode):
    """Stacked prefill of ragged prompts (one row range through every BitLinear, the scan
    per stream) against one prefill per stream: first tokens, logits and every layer's
    state bit for bit, also when fewer streams are prefilled than were reset. "odd"
    (hidden 100) takes the per-stream path (SIMD tails)."""
    from matmulfreellmcpu_amd import Engine, read_blob
    print(f"prefill_streams blob={name} mode={mode}", flush=True)
    blob = read_blob(blobs(name))
    V = blob.config.vocab_size
    rng = np.random.default_rng(5)
    prompts = [rng.integers(3, V, n) for n in (5, 12, 1, 7, 40, 3)]
    e = Engine(0)
    e.load_blob(blob, mode)
    B = len(prompts) + 2
    e.reset(B)
    want = [e.prefill(b, prompts[b], want_logits=True) for b in range(len(prompts))]
    want_state = e.state()
    e.reset(B)
    am, lg = e.prefill_streams(prompts, want_logits=True)
    got_state = e.state()
    for b in range(len(prompts)):
        assert int(am[b]) == want[b][0], b
        assert_bitexact(lg[b], want[b][1], f"stream {b} logits")
    assert_bitexact(got_state, want_state, "states after prefill")
    # the streams decode on from the stacked prefill exactly as from per-stream ones
    e2 = Engine(0)
    e2.load_blob(blob, mode)
    e2.reset(B)
    for b in range(len(prompts)):
        e2.prefill(b, prompts[b])
    tok = np.concatenate([am, [5, 6]]).astype(np.int64)
    for _ in range(3):
        a1, a2 = e.step(tok), e2.step(tok)
        np.testing.assert_array_equal(a1, a2)
        tok = a1
    assert_bitexact(e.state(), e2.state(), "states after decode steps")
    e.close()
    e2.close()


@pytest.mark.parametrize("mode", [FLOAT, FIXED])
def test_serve_stacked_matches_oracle(blobs, oracle, mode):
    """The serving path with the stacked prefill against the oracle's generate_serve."""
    from matmulfreellmcpu_amd import Engine, read_blob
    blob = read_blob(blobs("small"))
    om = oracle.model(blob)
    rng = np.random.default_rng(19)
    V = blob.config.vocab_size
    prompts = [rng.integers(3, V, n) for n in (9, 1, 33, 4)]
    want = om.generate_serve(prompts, 6, mode)
    e = Engine(0)
    e.load_blob(blob, mode)
    e.reset(len(prompts))
    streams = [list(p) + [int(t)] for p, t in zip(prompts, e.prefill_streams(prompts))]
    for _ in range(5):
        nxt = e.step([s[-1] for s in streams])
        for b in range(len(prompts)):
            streams[b].append(int(nxt[b]))
    for b in range(len(prompts)):
        np.testing.assert_array_equal(np.array(streams[b]), want[b])
    e.close()


@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
def test_serve_kgroups_matches_oracle(blobs, oracle, mode):
    """Serving steps of 56 streams whose MLP gate GEMM (6144 columns) runs as K-groups with
    the swiglu-pair epilogue after the LDS reduction (integer modes), or on 32 x 64 tiles of
    the 32x32 fp32 matrix-core instruction (float)."""
    from matmulfreellmcpu_amd import Engine, read_blob
    blob = read_blob(blobs("wide"))
    om = oracle.model(blob)
    rng = np.random.default_rng(23)
    prompts = [rng.integers(3, blob.config.vocab_size, 1 + (7 * b) % 12) for b in range(56)]
    print(f"serve k-groups mode={mode}", flush=True)
    want = om.generate_serve(prompts, 5, mode)
    e = Engine(0)
    e.load_blob(blob, mode)
    e.reset(len(prompts))
    streams = [list(p) + [int(t)] for p, t in zip(prompts, e.prefill_streams(prompts))]
    for _ in range(4):
        nxt = e.step([s[-1] for s in streams])
        for b in range(len(prompts)):
            streams[b].append(int(nxt[b]))
    for b in range(len(prompts)):
        np.testing.assert_array_equal(np.array(streams[b]), want[b])
    e.close()


@pytest.mark.parametrize("mode", [FLOAT, FIXED])
def test_generate_370m(blobs, oracle, mode):
    """Full 370M shape: 16-token prompt, 32 greedy tokens, bit-exact state."""
    from matmulfreellmcpu_amd import Engine, read_blob
    blob = read_blob(blobs("s0"))
    om = oracle.model(blob)
    ids = np.random.default_rng(0).integers(3, 32000, 16)
    want, wst = om.generate(ids, 32, mode, want_state=True)
    e = Engine(0)
    e.load_blob(blob, mode)
    np.testing.assert_array_equal(e.generate(ids, 32), want)
    assert_bitexact(e.state()[:, 0, :], wst, "370M final state")
    e.close()


def test_time_step_runs_the_step(blobs):
    """mmf_model_time_step launches the serving step kernel by kernel: one timed step
    (warmup 0, reps 1) leaves the streams exactly where mmf_model_step with the same tokens
    does (states and the next step's ids bit for bit), and reports time in the GEMM kinds."""
    from matmulfreellmcpu_amd import Engine, FIXED_Q510, read_blob
    print("time_step", flush=True)
    blob = read_blob(blobs("small"))
    rng = np.random.default_rng(8)
    prompts = [rng.integers(3, blob.config.vocab_size, 9) for _ in range(4)]
    t1, t2, t3 = (rng.integers(3, blob.config.vocab_size, 4) for _ in range(3))
    outs = []
    for timed in (False, True):
        e = Engine(0)
        e.load_blob(blob, FIXED_Q510)
        e.reset(4)
        e.prefill_streams(prompts)
        e.step(t1)
        if timed:
            k = e.time_step_kinds(t2, warmup=0, reps=1)
            assert all(v >= 0 for v in k.values()) and k["gemm_ifg"] > 0 and k["gemm_down"] > 0, k
        else:
            e.step(t2)
        ids = e.step(t3)
        outs.append((ids, e.state()))
        e.close()
    assert np.array_equal(outs[0][0], outs[1][0])
    assert_bitexact(outs[1][1], outs[0][1], "states after a timed step")
