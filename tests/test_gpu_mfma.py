"""The matrix-core (int8 MFMA) GEMM of the integer modes against the CPU restatement.

Row counts of 32 and more take the MFMA kernel (fewer take the dot-product kernel); the
results must be bit-exact: int32 accumulators, fp32 outputs, per-layer traces, streams.
"""
import numpy as np
import pytest

from conftest import assert_bitexact
from test_gpu_parity import Dev, eng  # noqa: F401  (module fixture)

pytestmark = pytest.mark.gpu

FLOAT, FIXED, INT8 = 0, 1, 2

SHAPES = [(32, 256, 128), (65, 100, 40), (130, 1024, 333), (300, 2816, 96), (64, 13, 5), (257, 2048, 512)]


@pytest.mark.parametrize("rows,K,N", SHAPES)
@pytest.mark.parametrize("mode", [FIXED, INT8])
def test_bitlinear_rows(eng, oracle, rows, K, N, mode):  # noqa: F811
    print(f"mfma bitlinear rows={rows} K={K} N={N} mode={mode}", flush=True)
    rng = np.random.default_rng(rows * 7 + K + N + mode)
    x = (rng.standard_normal((rows, K)) * 2).astype(np.float32)
    x[rows // 3] *= 40.0  # saturating Q5.10 codes in one row
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
    assert_bitexact(dout.get(), want["out"], f"bitlinear out mode {mode}")


# 8-32 rows on 32 x 64 tiles of eight K-groups (the row tile partly past the last row):
# K up to 4096, and over 16 rows up to 6912 with at least 32 tiles (16 x 5632 x 2048 takes
# the K split); with int32 accumulators (the general
# K-group sum and epilogue) and without (where the whole tile is in range: the shared one).
@pytest.mark.parametrize("rows,K,N", [(8, 1024, 1024), (12, 2048, 640), (16, 5632, 2048), (24, 6912, 2560),
                                      (31, 4096, 2112), (32, 2560, 2560)])
@pytest.mark.parametrize("mode", [FIXED, INT8])
@pytest.mark.parametrize("with_acc", [True, False])
def test_kgroup_few_rows(eng, oracle, rows, K, N, mode, with_acc):  # noqa: F811
    print(f"k-group few-row bitlinear rows={rows} K={K} N={N} mode={mode} acc={with_acc}", flush=True)
    rng = np.random.default_rng(rows * 11 + K + N + mode)
    x = (rng.standard_normal((rows, K)) * 2).astype(np.float32)
    x[rows // 3] *= 40.0  # saturating Q5.10 codes in one row
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    sw = float(np.float32(1.0 / 0.0157))
    want = oracle.bitlinear(x, nw, wq, sw, 1e-6, mode)
    pid = eng.register_proj(wq, sw, nw)
    dx, dout = Dev(eng, x), Dev(eng, shape=(rows, N))
    dacc = Dev(eng, shape=(rows, N), dtype=np.int32) if with_acc else None
    eng.bitlinear(pid, dx.ptr, dout.ptr, rows, mode=mode, acc=dacc.ptr if with_acc else None)
    eng.sync()
    if with_acc:
        np.testing.assert_array_equal(dacc.get(), want["acc"])
    assert_bitexact(dout.get(), want["out"], f"k-group few-row bitlinear out mode {mode}")


# Many-row Float and FixedQ510 prologues of long rows take the half-row LDS kernel (nb >=
# 512; Int8Absmax keeps the whole-row kernel): 4100 (pass B is only the tail group), 4231 (a
# 7-element tail; K % 4 != 0 takes the general prologue), 5632 and 6912 (the MLP down widths:
# 3 and 4 groups per thread), 4104 (one position past pass A, chain rows padded to 16).
@pytest.mark.parametrize("K", [4100, 4231, 4104, 5632, 6912])
@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
def test_bitlinear_long_rows(eng, oracle, K, mode):  # noqa: F811
    rows, N = 600, 64
    print(f"long-row bitlinear rows={rows} K={K} N={N} mode={mode}", flush=True)
    rng = np.random.default_rng(K * 3 + mode)
    x = (rng.standard_normal((rows, K)) * 2).astype(np.float32)
    x[rows // 3] *= 40.0  # saturating Q5.10 codes in one row
    x[rows // 2, : K // 2] = 0.0  # a row whose first half is zero
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


def test_cluster_rows(eng, oracle):  # noqa: F811
    rng = np.random.default_rng(55)
    rows, K, N = 70, 512, 160
    x = rng.standard_normal((rows, K)).astype(np.float32)
    pids, wants = [], []
    for j in range(3):
        nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
        wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
        pids.append(eng.register_proj(wq, 30.0 + j, nw))
        wants.append(oracle.bitlinear(x, nw, wq, 30.0 + j, 1e-6, FIXED)["out"])
    dx = Dev(eng, x)
    outs = [Dev(eng, shape=(rows, N)) for _ in range(3)]
    eng.bitlinear_cluster(pids, dx.ptr, [o.ptr for o in outs], rows, mode=FIXED)
    eng.sync()
    for o, w in zip(outs, wants):
        assert_bitexact(o.get(), w, "cluster")


@pytest.mark.parametrize("b,K,N", [(64, 1024, 256), (200, 2816, 64), (33, 13, 5)])
def test_ternary_matmul_rows(eng, oracle, b, K, N):  # noqa: F811
    rng = np.random.default_rng(b * 3 + K)
    x = rng.integers(-32768, 32768, (b, K)).astype(np.int32)
    x[0, :] = -32768  # extreme codes
    x[1, :] = 32767
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    pid = eng.register_proj(wq, 1.0)
    dx, dacc = Dev(eng, x), Dev(eng, shape=(b, N), dtype=np.int32)
    eng.ternary_matmul(pid, dx.ptr, dacc.ptr, b)
    eng.sync()
    np.testing.assert_array_equal(dacc.get(), oracle.ternary_matmul(x, wq))


@pytest.mark.parametrize("name", ["small", "odd"])
@pytest.mark.parametrize("mode", [FIXED, INT8])
def test_long_prefill_trace(blobs, oracle, name, mode):
    from matmulfreellmcpu_amd import Engine, read_blob
    print(f"mfma prefill trace blob={name} mode={mode}", flush=True)
    blob = read_blob(blobs(name))
    om = oracle.model(blob)
    ids = np.random.default_rng(77).integers(3, blob.config.vocab_size, 150)
    wh, wst, wtr = om.trace(ids, mode)
    e = Engine(0)
    e.load_blob(blob, mode)
    h, st, tr = e.trace(ids)
    for l in range(blob.config.num_hidden_layers):
        for k, nm in enumerate(("i", "f", "g", "scan", "recur")):
            assert_bitexact(tr[l, k], wtr[l, k], f"layer {l} {nm}")
        assert_bitexact(h[l], wh[l], f"layer {l} h")
        assert_bitexact(st[l], wst[l], f"layer {l} state")
    want, wstate = om.generate(ids, 8, mode, want_state=True)
    np.testing.assert_array_equal(e.generate(ids, 8), want)
    assert_bitexact(e.state()[:, 0, :], wstate, "state after long-prompt generate")
    e.close()


def test_serve_many_streams(blobs, oracle):
    """40 streams: the batched decode steps take the MFMA kernel."""
    from matmulfreellmcpu_amd import Engine, read_blob
    blob = read_blob(blobs("small"))
    om = oracle.model(blob)
    rng = np.random.default_rng(19)
    prompts = [rng.integers(3, blob.config.vocab_size, int(n)) for n in rng.integers(1, 40, 40)]
    want = om.generate_serve(prompts, 6, FIXED)
    e = Engine(0)
    e.load_blob(blob, FIXED)
    e.reset(len(prompts))
    streams = [list(p) for p in prompts]
    for b, p in enumerate(prompts):
        streams[b].append(e.prefill(b, p))
    for _ in range(5):
        nxt = e.step([s[-1] for s in streams])
        for b in range(len(prompts)):
            streams[b].append(int(nxt[b]))
    for b in range(len(prompts)):
        np.testing.assert_array_equal(np.array(streams[b]), want[b])
    e.close()
