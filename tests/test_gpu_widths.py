"""Parity at the production widths: the kernel variants that the 1.3B and 2.7B shapes and
the full BitLinear op sweep select, against the CPU restatement, bit for bit.

Two-layer blobs with the real widths and vocabulary (hidden 2048 / intermediate 5632 and
hidden 2560 / intermediate 6912, vocab 32000) reach what the smaller test blobs cannot:
  - single-row decode kernels with 8 and 16 chain positions per thread, and the lm_head
    whose blocks stride over several 16-output groups (hidden > 1024);
  - integer matrix-core tiles 4 waves wide (launches of >= 256 tiles: 2048-row prefills,
    8192- and 16384-row stacked serving prefills, the op sweep at M = 2048);
  - row prologues over 5632- and 6912-wide rows (7 float4 per thread in 256-thread blocks)
    and 1024-thread serving prologues with 2 float4 per thread;
  - the fp32 matrix-core tiles at the prefill shapes of the float mode.
"""
import numpy as np
import pytest

from conftest import assert_bitexact
from test_gpu_parity import Dev, eng  # noqa: F401  (module fixture)

pytestmark = pytest.mark.gpu

FLOAT, FIXED, INT8 = 0, 1, 2


def _engine(blob, mode):
    from matmulfreellmcpu_amd import Engine
    e = Engine(0)
    e.load_blob(blob, mode)
    return e


@pytest.mark.parametrize("name", ["h2048", "h2560"])
@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
def test_generate_widths(blobs, oracle, name, mode):
    """B=1 greedy generate, 16-token prompt and 32 new tokens: the id stream and the final
    recurrent state of every layer."""
    from matmulfreellmcpu_amd import read_blob
    print(f"generate widths blob={name} mode={mode}", flush=True)
    blob = read_blob(blobs(name))
    om = oracle.model(blob)
    ids = np.random.default_rng(101).integers(3, 32000, 16)
    want, wst = om.generate(ids, 32, mode, want_state=True)
    e = _engine(blob, mode)
    np.testing.assert_array_equal(e.generate(ids, 32), want)
    assert_bitexact(e.state()[:, 0, :], wst, f"{name} final state")
    e.close()


@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
def test_prefill_trace_2048(blobs, oracle, mode):
    """A 2048-token prompt on the 1.3B widths: every layer's i, gated f, g, scan input,
    recurrence output, h and state."""
    from matmulfreellmcpu_amd import read_blob
    print(f"prefill trace 2048 mode={mode}", flush=True)
    blob = read_blob(blobs("h2048"))
    om = oracle.model(blob)
    ids = np.random.default_rng(7).integers(3, 32000, 2048)
    wh, wst, wtr = om.trace(ids, mode)
    e = _engine(blob, mode)
    h, st, tr = e.trace(ids)
    e.close()
    for l in range(blob.config.num_hidden_layers):
        for k, nm in enumerate(("i", "f", "g", "scan", "recur")):
            assert_bitexact(tr[l, k], wtr[l, k], f"layer {l} {nm}")
        assert_bitexact(h[l], wh[l], f"layer {l} h")
        assert_bitexact(st[l], wst[l], f"layer {l} state")


SWEEP_KN = [(1024, 1024), (1024, 5632), (2816, 1024), (2048, 11264), (5632, 2048)]


@pytest.mark.parametrize("M", [1, 16, 256, 2048])
@pytest.mark.parametrize("K,N", SWEEP_KN)
def test_op_sweep_int8(eng, oracle, M, K, N):  # noqa: F811
    """The BitLinear op sweep (Int8Absmax, RMSNorm eps 1e-6, unit norm weights, x ~ N(0,1)):
    int32 accumulators and outputs at every (M, K, N)."""
    print(f"op sweep int8 M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M + 3 * K + 7 * N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = np.ones(K, np.float32)
    wq = rng.choice(np.array([-1, 0, 1], np.int8), size=(N, K), p=[0.345, 0.31, 0.345])
    sw = float(np.float32(1.0 / 0.0160))
    want = oracle.bitlinear(x, nw, wq, sw, 1e-6, INT8)
    pid = eng.register_proj(wq, sw, nw)
    dx, dout = Dev(eng, x), Dev(eng, shape=(M, N))
    dacc = Dev(eng, shape=(M, N), dtype=np.int32)
    eng.bitlinear(pid, dx.ptr, dout.ptr, M, mode=INT8, acc=dacc.ptr)
    eng.sync()
    np.testing.assert_array_equal(dacc.get(), want["acc"])
    assert_bitexact(dout.get(), want["out"], f"int8 out M={M} K={K} N={N}")


@pytest.mark.parametrize("mode", [FLOAT, FIXED, INT8])
@pytest.mark.parametrize("K,N,off", [(1024, 1024, 0), (2560, 2560, 0), (6912, 2560, 0), (2048, 512, 1), (1000, 64, 0)])
def test_single_row_bitlinear(eng, oracle, mode, K, N, off):  # noqa: F811
    """One row of one projection: at the model widths (K = 256 RC, 16-byte aligned row) the
    integer modes run norm, encoding and GEMV in one launch; a row one float off alignment,
    a width of no register chain (K = 1000) and float mode take the two-launch path. Every
    case against the oracle, with the int32 accumulators, and rows that saturate Q5.10."""
    print(f"single row mode={mode} K={K} N={N} off={off}", flush=True)
    rng = np.random.default_rng(K * 7 + N + mode)
    x = (rng.standard_normal((1, K)) * 2).astype(np.float32)
    x[0, :: 97] *= 1e4  # large values: codes at the Q5.10 clamp
    nw = (1 + 0.2 * rng.standard_normal(K)).astype(np.float32)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    sw = float(np.float32(1.0 / 0.0157))
    want = oracle.bitlinear(x, nw, wq, sw, 1e-6, mode)
    pid = eng.register_proj(wq, sw, nw)
    buf = np.zeros((1, K + 4), np.float32)
    buf[0, off:off + K] = x[0]
    dx, dout = Dev(eng, buf), Dev(eng, shape=(1, N))
    dacc = Dev(eng, shape=(1, N), dtype=np.int32)
    eng.bitlinear(pid, dx.ptr + 4 * off, dout.ptr, 1, mode=mode, acc=None if mode == FLOAT else dacc.ptr)
    eng.sync()
    if mode != FLOAT:
        np.testing.assert_array_equal(dacc.get(), want["acc"])
    assert_bitexact(dout.get(), want["out"], f"single row mode={mode} K={K} N={N}")


@pytest.mark.parametrize("K,N", [(2048, 11264), (5632, 2048)])
def test_op_sweep_fixed_2048(eng, oracle, K, N):  # noqa: F811
    """The two matrix-core-bound sweep shapes at M = 2048 in FixedQ510 (both code planes)."""
    rng = np.random.default_rng(K + N)
    x = (rng.standard_normal((2048, K)) * 3).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    sw = float(np.float32(1.0 / 0.0157))
    want = oracle.bitlinear(x, nw, wq, sw, 1e-6, FIXED)
    pid = eng.register_proj(wq, sw, nw)
    dx, dout = Dev(eng, x), Dev(eng, shape=(2048, N))
    dacc = Dev(eng, shape=(2048, N), dtype=np.int32)
    eng.bitlinear(pid, dx.ptr, dout.ptr, 2048, mode=FIXED, acc=dacc.ptr)
    eng.sync()
    np.testing.assert_array_equal(dacc.get(), want["acc"])
    assert_bitexact(dout.get(), want["out"], f"fixed out K={K} N={N}")


@pytest.mark.parametrize("K,N", [(2048, 11264), (5632, 2048)])
def test_ternary_matmul_2048(eng, oracle, K, N):  # noqa: F811
    """TernaryBackend::matmul_batch with b = 2048 int16-range codes at the sweep shapes."""
    rng = np.random.default_rng(3 * K + N)
    x = rng.integers(-32768, 32768, (2048, K)).astype(np.int32)
    x[0, :] = -32768
    x[1, :] = 32767
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    pid = eng.register_proj(wq, 1.0)
    dx, dacc = Dev(eng, x), Dev(eng, shape=(2048, N), dtype=np.int32)
    eng.ternary_matmul(pid, dx.ptr, dacc.ptr, 2048)
    eng.sync()
    np.testing.assert_array_equal(dacc.get(), oracle.ternary_matmul(x, wq))


def _serve(blob, mode, prompts, steps):
    e = _engine(blob, mode)
    e.reset(len(prompts))
    streams = [list(p) + [int(t)] for p, t in zip(prompts, e.prefill_streams(prompts))]
    for _ in range(steps):
        nxt = e.step([s[-1] for s in streams])
        for b in range(len(prompts)):
            streams[b].append(int(nxt[b]))
    st = e.state()
    e.close()
    return streams, st


@pytest.mark.parametrize("mode", [FIXED, FLOAT])
def test_serve_2560_64_streams(blobs, oracle, mode):
    """64 streams of 128-token prompts on the 2.7B widths: stacked prefill (8192 rows) and 4
    batched steps; every stream's ids and the final recurrent state against the oracle's
    generate_serve."""
    from matmulfreellmcpu_amd import read_blob
    print(f"serve h2560 64 streams mode={mode}", flush=True)
    blob = read_blob(blobs("h2560"))
    om = oracle.model(blob)
    rng = np.random.default_rng(64 + mode)
    prompts = [rng.integers(3, 32000, 128) for _ in range(64)]
    want, wst = om.generate_serve(prompts, 5, mode, want_state=True)
    got, st = _serve(blob, mode, prompts, 4)
    for b in range(64):
        np.testing.assert_array_equal(np.array(got[b]), want[b], err_msg=f"stream {b}")
    assert_bitexact(st, wst, "recurrent state of every layer and stream")


def test_serve_2048_32_streams_fixed(blobs, oracle):
    """32 FixedQ510 streams on the 1.3B widths: 512-token prompts stacked into 16384 rows, then
    4 batched steps; every stream's ids and the final recurrent state of every layer against
    the oracle's generate_serve."""
    from matmulfreellmcpu_amd import read_blob
    print("serve h2048 32 streams fixed", flush=True)
    blob = read_blob(blobs("h2048"))
    om = oracle.model(blob)
    rng = np.random.default_rng(32)
    prompts = [rng.integers(3, 32000, 512) for _ in range(32)]
    want, wst = om.generate_serve(prompts, 5, FIXED, want_state=True)
    got, st = _serve(blob, FIXED, prompts, 4)
    for b in range(32):
        np.testing.assert_array_equal(np.array(got[b]), want[b], err_msg=f"stream {b}")
    assert_bitexact(st, wst, "recurrent state of every layer and stream")
