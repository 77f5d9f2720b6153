"""Pins the CPU restatement (oracle/mmf_oracle.c) that the GPU parity tests use as checker.

Three independent anchors, so a plausible mistake in the restatement (a dropped FMA, a
different summation order, a wrong tail rule, a transposed operand) fails at least one:
  1. golden vectors written by the reference engine compiled from its own sources
     (tests/golden/make_golden.py), always available;
  2. the compiled reference itself (oracle/_ref) on fresh random inputs, where built;
  3. closed forms: integer dot products by brute force, the int8 absmax formula,
     exact-product special cases of the recurrence, the hsum association, argmax ties.
"""
import hashlib
import os

import numpy as np
import pytest

from conftest import assert_bitexact, bits

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FLOAT, FIXED, INT8 = 0, 1, 2


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


# ---------------------------------------------------------------------------------------
# 1. golden vectors
# ---------------------------------------------------------------------------------------
def test_golden_primitives(oracle):
    g = load("prims.npz")
    x, b = g["x"], g["b"]
    assert_bitexact(oracle.sigmoid(x), g["sigmoid"], "sigmoid")
    assert_bitexact(oracle.silu(x), g["silu"], "silu")
    assert_bitexact(oracle.swiglu(x, b), g["swiglu"], "swiglu")
    for n, want in zip(g["sumsq_n"], g["sumsq"]):
        assert bits(oracle.sumsq(g["sumsq_x"][:n])) == bits(want), f"sumsq n={n}"
    np.testing.assert_array_equal(oracle.quant_q510(g["quant_y"]), g["quant_q510"])
    import ctypes as C
    for n, want in zip(g["dot_n"], g["dot_f32"]):
        y = np.ascontiguousarray(g["dot_y"][:n])
        w = np.ascontiguousarray(g["dot_w"][:n])
        got = oracle.lib.mo_ternary_dot_f32(y.ctypes.data_as(C.POINTER(C.c_float)),
                                            w.ctypes.data_as(C.POINTER(C.c_int8)), int(n))
        assert bits(got) == bits(want), f"ternary_dot_f32 n={n}"


def test_golden_bitlinear(oracle):
    g = load("bitlinear.npz")
    for ci in range(int(g["ncases"])):
        x, nw, wq, sw = g[f"c{ci}_x"], g[f"c{ci}_normw"], g[f"c{ci}_wq"], float(g[f"c{ci}_scale"])
        for mode, nm in ((FLOAT, "float"), (FIXED, "fixed")):
            r = oracle.bitlinear(x, nw, wq, sw, 1e-6, mode)
            assert_bitexact(r["norm"], g[f"c{ci}_{nm}_norm"], f"case {ci} {nm} norm")
            assert_bitexact(r["out"], g[f"c{ci}_{nm}_out"], f"case {ci} {nm} out")


@pytest.fixture(scope="module")
def tiny_blob(tmp_path_factory):
    from matmulfreellmcpu_amd import make_blob, read_blob
    import conftest
    conftest._mkblob_bin()
    g = load("model_tiny.npz")
    p = str(tmp_path_factory.mktemp("gold") / "tiny.mmfree")
    make_blob(p, preset="tiny", seed=20261201, random_norms=True, random_lb=True)
    sha = hashlib.sha256(open(p, "rb").read()).hexdigest()
    assert sha == str(g["blob_sha256"]), "mmfree-mkblob no longer reproduces the fixture blob"
    return p, read_blob(p), g


@pytest.mark.parametrize("mode,nm", [(FLOAT, "float"), (FIXED, "fixed")])
def test_golden_model(oracle, tiny_blob, mode, nm):
    _, blob, g = tiny_blob
    om = oracle.model(blob)
    ids = g["ids"]
    got, st = om.generate(ids, 24, mode, want_state=True)
    np.testing.assert_array_equal(got, g[f"{nm}_greedy"])
    assert_bitexact(st, g[f"{nm}_state"], "final state")
    assert_bitexact(om.forward(ids, mode), g[f"{nm}_forward"], "forward logits")
    h, st, tr = om.trace(ids, mode)
    assert_bitexact(h, g[f"{nm}_trace_h"], "trace h")
    assert_bitexact(st, g[f"{nm}_trace_state"], "trace state")
    assert_bitexact(tr, g[f"{nm}_trace_int"], "trace internals")
    prompts = [g[f"serve_prompt{i}"] for i in range(4)]
    for i, s in enumerate(om.generate_serve(prompts, 8, mode)):
        np.testing.assert_array_equal(s, g[f"{nm}_serve{i}"])


# ---------------------------------------------------------------------------------------
# 2. against the compiled reference (random inputs)
# ---------------------------------------------------------------------------------------
def test_ref_random_primitives(oracle, ref):
    rng = np.random.default_rng(99)
    for n in (1, 7, 8, 15, 16, 33, 8192 + 7, 20001):
        x = (rng.standard_normal(n) * rng.uniform(0.1, 60)).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        assert bits(oracle.sumsq(x)) == bits(ref.sumsq(x)), n
        assert_bitexact(oracle.sigmoid(x), ref.sigmoid(x), f"sigmoid {n}")
        assert_bitexact(oracle.silu(x), ref.silu(x), f"silu {n}")
        assert_bitexact(oracle.swiglu(x, b), ref.swiglu(x, b, chunked=False), f"swiglu {n}")
        np.testing.assert_array_equal(oracle.quant_q510(x * 500), ref.quant_q510(x * 500))


@pytest.mark.parametrize("rows,K,N", [(1, 64, 64), (4, 1024, 96), (2, 2816, 33), (3, 13, 9)])
def test_ref_random_bitlinear(oracle, ref, rows, K, N):
    rng = np.random.default_rng(rows * K + N)
    x = (rng.standard_normal((rows, K)) * 3).astype(np.float32)
    nw = (1 + 0.2 * rng.standard_normal(K)).astype(np.float32)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    for mode in (FLOAT, FIXED):
        a = oracle.bitlinear(x, nw, wq, 53.7, 1e-6, mode)
        r = ref.bitlinear(x, nw, wq, 53.7, 1e-6, mode)
        assert_bitexact(a["out"], r["out"], f"mode {mode}")
        assert_bitexact(a["norm"], r["norm"], f"norm mode {mode}")
    xq = rng.integers(-32768, 32768, (rows, K)).astype(np.int32)
    np.testing.assert_array_equal(oracle.ternary_matmul(xq, wq), ref.ternary_matmul(xq, wq))


def test_ref_cluster_equals_single(ref):
    """bitlinear_cluster is bit-identical to separate bitlinear calls (kernels.hpp:46-50)."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    nws = [(1 + 0.1 * rng.standard_normal(128)).astype(np.float32) for _ in range(3)]
    wqs = [rng.integers(-1, 2, (40, 128)).astype(np.int8) for _ in range(3)]
    outs = ref.bitlinear_cluster(x, nws, wqs, [30.0, 31.0, 32.0], 1e-6)
    for j in range(3):
        assert_bitexact(outs[j], ref.bitlinear(x, nws[j], wqs[j], 30.0 + j, 1e-6, FIXED)["out"], "cluster")


@pytest.mark.parametrize("mode", [FLOAT, FIXED])
def test_ref_model_odd_shapes(oracle, ref, blobs, mode):
    """hidden 100 (not a multiple of 8): every scalar-tail rule of the reference is exercised."""
    from matmulfreellmcpu_amd import read_blob
    p = blobs("odd")
    om = oracle.model(read_blob(p))
    rm = ref.model(p, mode)
    ids = np.array([5, 900, 17, 3, 64, 512, 999])
    np.testing.assert_array_equal(om.generate(ids, 16, mode), rm.generate(ids, 16))
    assert_bitexact(om.generate(ids, 16, mode, want_state=True)[1], rm.state(), "state")
    assert_bitexact(om.forward(ids, mode), rm.forward(ids), "forward")
    rm.close()


# ---------------------------------------------------------------------------------------
# 3. closed forms and invariants
# ---------------------------------------------------------------------------------------
def test_integer_dot_brute_force(oracle):
    rng = np.random.default_rng(1)
    x = rng.integers(-32768, 32768, (3, 777)).astype(np.int32)
    w = rng.integers(-1, 2, (50, 777)).astype(np.int8)
    want = (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.int32)
    np.testing.assert_array_equal(oracle.ternary_matmul(x, w), want)


def test_int8_absmax_closed_form(oracle):
    """Int8Absmax mode = tools/reference.py:131-135,180-184 in fp32."""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((4, 96)) * 2).astype(np.float32)
    nw = np.ones(96, np.float32)
    wq = rng.integers(-1, 2, (24, 96)).astype(np.int8)
    sw = np.float32(47.0)
    r = oracle.bitlinear(x, nw, wq, float(sw), 1e-6, INT8)
    y = r["norm"]
    amax = np.abs(y).max(axis=1, keepdims=True)
    sa = (np.float32(127.0) / np.maximum(amax, np.float32(1e-5))).astype(np.float32)
    q = np.clip(np.rint(y * sa), -128, 127).astype(np.int64)
    np.testing.assert_array_equal(r["scale_a"], sa[:, 0])
    np.testing.assert_array_equal(r["codes"], q)
    acc = q @ wq.astype(np.int64).T
    np.testing.assert_array_equal(r["acc"], acc)
    want = acc.astype(np.float32) / (sw * sa)
    assert_bitexact(r["out"], want.astype(np.float32), "int8 out")


def test_int8_absmax_known_answers(oracle):
    """Hand-computed vectors for tools/reference.py:131-135,180-184: x = ones and eps = 0 give
    rstd = 1 exactly, so y = normw; max|y| = 127/64 gives scale_a = 64 exactly. y*scale_a hits
    +-2.5 (round half to even -> +-2, half away from zero would give +-3), 3.5 (-> 4) and
    +-127; one-hot weight rows make acc = the codes, and acc / (scale_w * scale_a) with
    scale_w = 2 gives exact eighths of a sixteenth."""
    y = np.array([127 / 64, -127 / 64, 2.5 / 64, -2.5 / 64, 3.5 / 64, 0.0, 1 / 128, 40 / 64],
                 np.float32)
    x = np.ones((1, 8), np.float32)
    wq = np.eye(8, dtype=np.int8)
    r = oracle.bitlinear(x, y, wq, 2.0, 0.0, INT8)
    assert r["scale_a"][0] == np.float32(64.0)
    np.testing.assert_array_equal(r["codes"][0], [127, -127, 2, -2, 4, 0, 0, 40])
    np.testing.assert_array_equal(r["acc"][0], [127, -127, 2, -2, 4, 0, 0, 40])
    np.testing.assert_array_equal(r["out"][0], np.array([127, -127, 2, -2, 4, 0, 0, 40], np.float32) / 128)


def test_fixed_codes_and_acc_closed_form(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 64)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(64)).astype(np.float32)
    wq = rng.integers(-1, 2, (8, 64)).astype(np.int8)
    r = oracle.bitlinear(x, nw, wq, 40.0, 1e-6, FIXED)
    q = np.clip(np.rint(r["norm"] * np.float32(1024)), -32768, 32767).astype(np.int64)
    np.testing.assert_array_equal(r["codes"], q)
    np.testing.assert_array_equal(r["acc"], q @ wq.astype(np.int64).T)
    inv = np.float32(1.0) / (np.float32(1024.0) * np.float32(40.0))
    assert_bitexact(r["out"], r["acc"].astype(np.float32) * inv, "dequant")


def test_rmsnorm_closed_form(oracle):
    """With sumsq exact (small integers), rstd = 1/sqrt(ss/n + eps) and y = (x*rstd)*w."""
    x = np.array([[1, 2, 3, 4, 5, 6, 7, 8, -1, -2, 3, 1, 0, 2, 2, 1]], np.float32)
    w = np.linspace(0.5, 2, 16).astype(np.float32)
    ss = np.float32((x.astype(np.float64) ** 2).sum())
    rstd = np.float32(1.0) / np.sqrt(ss / np.float32(16) + np.float32(1e-6))
    assert_bitexact(oracle.rmsnorm(x, w, 1e-6), (x * rstd) * w, "rmsnorm")


def test_hsum_association(oracle):
    """((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)): cancellation makes other trees differ."""
    a = np.array([1e8, 1.0, 3.0, 5.0, -1e8, 1.0, 7.0, 1.0], np.float32)
    f = np.float32
    want = ((f(a[0]) + f(a[4])) + (f(a[1]) + f(a[5]))) + ((f(a[2]) + f(a[6])) + (f(a[3]) + f(a[7])))
    assert bits(oracle.hsum8(a)) == bits(want)
    seq = f(0)
    for v in a:
        seq = f(seq + f(v))
    assert bits(want) != bits(seq), "the test input no longer separates the two orders"


def test_lane_order_of_dot(oracle):
    """Lane j sums k = j (mod 8) in order: a value that cancels only within a lane."""
    y = np.zeros(16, np.float32)
    y[0], y[8], y[1] = 1e8, -1e8, 1.0  # lane 0 cancels to 0; lane 1 holds 1
    w = np.ones(16, np.int8)
    import ctypes as C
    got = oracle.lib.mo_ternary_dot_f32(y.ctypes.data_as(C.POINTER(C.c_float)),
                                        w.ctypes.data_as(C.POINTER(C.c_int8)), 16)
    assert got == 1.0
    y2 = y.copy()
    y2[8], y2[9] = 0.0, -1e8  # now -1e8 sits in lane 1 with the 1.0: absorbs it
    got2 = oracle.lib.mo_ternary_dot_f32(y2.ctypes.data_as(C.POINTER(C.c_float)),
                                         w.ctypes.data_as(C.POINTER(C.c_int8)), 16)
    assert got2 == 0.0


def test_scan_exact_products(oracle):
    """f in {0, 0.5, 1}: every product is exact, so fma(f, s, i) = f*s + i in numpy."""
    rng = np.random.default_rng(5)
    T, D = 40, 24
    f = rng.choice(np.array([0.0, 0.5, 1.0], np.float32), (T, D))
    i = rng.integers(-8, 8, (T, D)).astype(np.float32)
    st = rng.integers(-4, 4, D).astype(np.float32)
    out, s = oracle.hgrn_scan(i, f, st)
    ref_s = st.copy()
    for t in range(T):
        ref_s = f[t] * ref_s + i[t]
        np.testing.assert_array_equal(out[t], ref_s)
    np.testing.assert_array_equal(s, ref_s)


def test_activations_special_values(oracle):
    x = np.array([0.0, 200.0, -200.0, 88.3762626647949, -88.3762626647949] * 2, np.float32)
    sg = oracle.sigmoid(x)
    # the clamp at +-88.376 keeps 2^n finite (n = 127): sigmoid(-200) is a denormal, not 0
    assert sg[0] == 0.5 and sg[1] == 1.0 and 0.0 < sg[2] < 1e-38
    si = oracle.silu(x)
    assert si[0] == 0.0 and si[1] == 200.0 and -1e-35 < si[2] < 0.0
    z = np.linspace(-30, 30, 4001).astype(np.float32)
    np.testing.assert_allclose(oracle.sigmoid(z), 1 / (1 + np.exp(-z.astype(np.float64))), rtol=3e-7, atol=1e-30)


def test_quant_rounding_and_saturation(oracle):
    # 16 values on the SIMD body path, the 17th on the scalar tail
    y = np.zeros(17, np.float32)
    y[:5] = np.array([0.5, 1.5, 2.5, -0.5, -2.5], np.float32) / np.float32(1024)  # ties to even
    y[5:8] = np.array([40.0, -40.0, 3e9], np.float32)
    y[16] = np.float32(3e9)
    q = oracle.quant_q510(y)
    np.testing.assert_array_equal(q[:8], [0, 2, 2, 0, -2, 32767, -32768, -32768])  # body: huge -> INT_MIN
    assert q[16] == 32767  # the scalar tail saturates in float


def test_argmax_first_index(oracle):
    v = np.array([1.0, 3.0, 2.0, 3.0, -1.0], np.float32)
    assert oracle.argmax(v) == 1
    assert oracle.argmax(np.array([-0.0, 0.0], np.float32)) == 0


def test_serve_identical_prompts_equal_generate(oracle, blobs):
    """model.hpp:58-59: B identical prompts + greedy == single-stream generate."""
    from matmulfreellmcpu_amd import read_blob
    om = oracle.model(read_blob(blobs("tiny")))
    p = np.array([3, 17, 200, 45])
    for mode in (FLOAT, FIXED):
        single = om.generate(p, 10, mode)
        for s in om.generate_serve([p, p, p], 10, mode):
            np.testing.assert_array_equal(s, single)


def test_incremental_equals_recompute(oracle, blobs):
    """hgrn_model.cpp:312-314: the last decode logits equal forward() over the full prefix."""
    from matmulfreellmcpu_amd import read_blob
    om = oracle.model(read_blob(blobs("tiny")))
    p = np.array([3, 17, 200, 45, 7])
    for mode in (FLOAT, FIXED):
        stream, lg = om.generate(p, 6, mode, want_logits=True)
        full = om.forward(stream[:-1], mode)[-1]
        assert_bitexact(lg, full, "incremental vs recompute")
