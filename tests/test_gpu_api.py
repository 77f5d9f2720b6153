"""The drop-in C++ layer on the GPU.

1. The reference's own engine (compiled from its sources into oracle/_ref) with the MI355X
   TernaryBackend attached through its plugin seam, Model::set_backend (model.hpp:74-79 of
   the reference): FixedQ510 generation must give the same ids and the same recurrent state,
   bit for bit, as the reference's CPU run.
2. Our mmfree-cli (the reference CLI's flags, cpp/app/main.cpp:14-40) against the reference
   CLI: --print-ids streams (greedy and seeded sampling) and --logits-out bytes.
3. The mmfree C++ API (libmmfree.so, driven by tests/cpp/api_check.cpp): the kernels.hpp
   operators against the CPU restatement, Model::generate / generate_serve (greedy and
   sampled, with callbacks) against the reference Model.
"""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, assert_bitexact

pytestmark = pytest.mark.gpu

FLOAT, FIXED, INT8 = 0, 1, 2
CLI = os.path.join(ROOT, "matmulfreellmcpu_amd", "_lib", "mmfree-cli")
API_CHECK = os.path.join(ROOT, "tests", "cpp", "_build", "api_check")
REF_HIPBE_SO = os.path.join(ROOT, "oracle", "_ref", "libmmfree_ref_hipbe.so")


def _need(path):
    if not os.path.exists(path):
        pytest.skip(f"{os.path.relpath(path, ROOT)} not built")


def _run(cmd, timeout=120):
    print("run:", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, f"{cmd[0]} exit {r.returncode}: {r.stderr[-2000:]}"
    return r.stdout


# ---- 1. the reference Model with HipTernaryBackend -----------------------------------------

@pytest.fixture(scope="module")
def ref_hipbe():
    _need(REF_HIPBE_SO)
    from oracle.oracle import Ref
    r = Ref(REF_HIPBE_SO)
    r.lib.ref_model_ptr.restype = C.c_void_p
    r.lib.ref_model_ptr.argtypes = [C.c_void_p]
    r.lib.ref_hipbe_attach.restype = C.c_void_p
    r.lib.ref_hipbe_attach.argtypes = [C.c_void_p, C.c_int]
    r.lib.ref_model_weights.restype = C.c_void_p
    r.lib.ref_model_weights.argtypes = [C.c_void_p]
    r.lib.ref_hipbe_attach_registered.restype = C.c_void_p
    r.lib.ref_hipbe_attach_registered.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    r.lib.ref_hipbe_detach.restype = None
    r.lib.ref_hipbe_detach.argtypes = [C.c_void_p, C.c_void_p]
    return r


@pytest.mark.parametrize("name", ["tiny", "small", "odd"])
def test_reference_model_with_hip_backend_registered(ref_hipbe, blobs, name):
    """The registry deployment of the seam: every projection registered up front and the tag ->
    proj_id map handed to the reference's Model::set_backend (model.hpp:74-79)."""
    print(f"reference Model + HipTernaryBackend with the tag registry, blob={name}", flush=True)
    blob = blobs(name)
    rng = np.random.default_rng(43)
    ids = rng.integers(3, 1000, 9).astype(np.int64)
    cpu = ref_hipbe.model(blob, FIXED)
    want_ids = cpu.generate(ids, 12)
    want_state = cpu.state()
    prompts = [ids[:5], ids, ids[2:4]]
    want_serve = cpu.generate_serve(prompts, 6)
    gpu = ref_hipbe.model(blob, FIXED)
    be = ref_hipbe.lib.ref_hipbe_attach_registered(ref_hipbe.lib.ref_model_ptr(gpu.h),
                                                   ref_hipbe.lib.ref_model_weights(gpu.h), 0)
    assert be
    try:
        got_ids = gpu.generate(ids, 12)
        got_state = gpu.state()
        got_serve = gpu.generate_serve(prompts, 6)
    finally:
        ref_hipbe.lib.ref_hipbe_detach(ref_hipbe.lib.ref_model_ptr(gpu.h), be)
    np.testing.assert_array_equal(got_ids, want_ids)
    assert_bitexact(got_state, want_state, "recurrent state")
    for g, w in zip(got_serve, want_serve):
        np.testing.assert_array_equal(g, w)


@pytest.mark.parametrize("name", ["tiny", "small", "odd"])
def test_reference_model_with_hip_backend(ref_hipbe, blobs, name):
    print(f"reference Model + HipTernaryBackend blob={name}", flush=True)
    blob = blobs(name)
    rng = np.random.default_rng(41)
    ids = rng.integers(3, 1000, 9).astype(np.int64)
    cpu = ref_hipbe.model(blob, FIXED)
    want_ids = cpu.generate(ids, 12)
    want_state = cpu.state()
    gpu = ref_hipbe.model(blob, FIXED)
    be = ref_hipbe.lib.ref_hipbe_attach(ref_hipbe.lib.ref_model_ptr(gpu.h), 0)
    assert be
    try:
        got_ids = gpu.generate(ids, 12)
        got_state = gpu.state()
        # the serving path: batched matmuls (b = streams) through the same seam
        prompts = [ids[:5], ids, ids[2:4]]
        want_serve = cpu.generate_serve(prompts, 6)
        got_serve = gpu.generate_serve(prompts, 6)
    finally:
        ref_hipbe.lib.ref_hipbe_detach(ref_hipbe.lib.ref_model_ptr(gpu.h), be)
    np.testing.assert_array_equal(got_ids, want_ids)
    assert_bitexact(got_state, want_state, "recurrent state")
    for g, w in zip(got_serve, want_serve):
        np.testing.assert_array_equal(g, w)


# ---- 2. mmfree-cli against the reference CLI ----------------------------------------------

def _ref_cli():
    from oracle.oracle import REF_CLI
    _need(REF_CLI)
    return REF_CLI


CLI_CASES = [
    ("float", []),
    ("fixed", []),
    ("float", ["--temp", "0.8", "--top-k", "40", "--seed", "7"]),
    ("fixed", ["--temp", "1.1", "--seed", "123"]),
    ("fixed", ["--frac", "8"]),
]


@pytest.mark.parametrize("mode,extra", CLI_CASES)
def test_cli_ids_match_reference(blobs, tmp_path, mode, extra):
    _need(CLI)
    ref_cli = _ref_cli()
    blob = blobs("small")
    args = ["--blob", blob, "--ids", "5,17,400,3,99,1000", "--gen", "16", "--mode", mode, "--print-ids"] + extra
    ours = tmp_path / "ours.f32"
    theirs = tmp_path / "theirs.f32"
    got = _run([CLI] + args + ["--logits-out", str(ours)])
    want = _run([ref_cli] + args + ["--logits-out", str(theirs)])
    assert got == want
    assert len(got.split()) == 6 + 16
    assert_bitexact(np.fromfile(ours, np.float32), np.fromfile(theirs, np.float32), "--logits-out")


def test_cli_text_generation_matches_reference(blobs, tmp_path):
    """Text in, streamed text out (the reference CLI's main path): same bytes on stdout, with
    BOS, --no-bos, sampling, and an EOS stop (the tokenizer's EOS set to the first greedy
    token, so text generation stops right after it)."""
    _need(CLI)
    ref_cli = _ref_cli()
    from tok_util import make_tokenizer, write_mmtok
    blob = blobs("small")
    tok = str(tmp_path / "t.mmtok")
    pieces, merges = make_tokenizer(tok, seed=4)
    cases = [["--gen", "12", "--mode", "fixed", "the quick brown fox"],
             ["--gen", "12", "--mode", "float", "--no-bos", "café über"],
             ["--gen", "10", "--mode", "fixed", "--temp", "0.9", "--seed", "5", "once upon a time"],
             ["--gen", "6", "--mode", "float", "--show-ids", "hello world"]]
    for extra in cases:
        args = ["--blob", blob, "--tokenizer", tok] + extra
        a = subprocess.run([CLI] + args, capture_output=True, timeout=120)
        b = subprocess.run([ref_cli] + args, capture_output=True, timeout=120)
        assert a.returncode == b.returncode == 0, (extra, a.stderr[-500:], b.stderr[-500:])
        assert a.stdout == b.stdout, extra
        if "--show-ids" in extra:
            assert a.stderr == b.stderr
    first = _run([ref_cli, "--blob", blob, "--tokenizer", tok, "--gen", "1", "--mode", "fixed", "--print-ids",
                  "the quick brown fox"]).split()[-1]
    eos_tok = str(tmp_path / "e.mmtok")
    write_mmtok(eos_tok, pieces, merges, eos=int(first))
    args = ["--blob", blob, "--tokenizer", eos_tok, "--gen", "12", "--mode", "fixed", "--show-ids", "the quick brown fox"]
    a = subprocess.run([CLI] + args, capture_output=True, timeout=120)
    b = subprocess.run([ref_cli] + args, capture_output=True, timeout=120)
    assert a.returncode == b.returncode == 0
    assert a.stdout == b.stdout and a.stderr == b.stderr
    assert b"gen ids (1):" in a.stderr


def test_cli_errors_like_reference(blobs):
    _need(CLI)
    r = subprocess.run([CLI, "--no-such-flag"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "unknown arg" in r.stderr
    r = subprocess.run([CLI, "--blob", "/nonexistent.mmfree", "--ids", "1,2"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode != 0


def test_cli_bench_runs(blobs):
    _need(CLI)
    out = _run([CLI, "--blob", blobs("small"), "--ids", "5,6,7", "--gen", "8", "--bench", "--reps", "2",
                "--mode", "float"])
    assert "decode" in out and "  threads:       1\n" in out
    # --profile: the device time of the engine's kernels per op, in the reference's table
    for extra in (["--bench", "--reps", "2"], []):
        out = _run([CLI, "--blob", blobs("small"), "--ids", "5,6,7", "--gen", "8", "--mode", "fixed", "--profile"]
                   + extra)
        assert "op profile (" in out and "matmul (incl lm_head):" in out, out
        ops = {ln.split()[0] for ln in out.splitlines() if ln.startswith("  ") and len(ln.split()) == 5}
        assert {"matmul", "lm_head", "norm+quant", "embed"} <= ops, out


# ---- 3. the C++ API ------------------------------------------------------------------------

def _streams(path):
    with open(path) as f:
        return [np.array([int(t) for t in line.split()], np.int64) for line in f if line.strip()]


def test_cpp_api(blobs, oracle, ref, tmp_path):
    _need(API_CHECK)
    d = tmp_path
    rng = np.random.default_rng(2026)
    rows, K, N = 5, 200, 72
    x = (rng.standard_normal((rows, K)) * 1.5).astype(np.float32)
    nw = (1 + 0.2 * rng.standard_normal(K)).astype(np.float32)
    o2 = rng.standard_normal((rows, K)).astype(np.float32)
    wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
    scale = float(np.float32(1 / 0.0213))
    x.tofile(d / "x.f32")
    nw.tofile(d / "nw.f32")
    o2.tofile(d / "o.f32")
    wq.tofile(d / "wq.i8")
    fg = rng.uniform(0.05, 0.95, (rows, K)).astype(np.float32)
    fg.tofile(d / "f.f32")
    (d / "dims.txt").write_text(f"{rows} {K} {N} {scale!r}\n")
    prompts = [[5, 17, 400, 3, 99], [7], [1000, 2, 2, 31]]
    (d / "prompts.txt").write_text("\n".join(" ".join(map(str, p)) for p in prompts) + "\n")
    blob = blobs("small")
    out = _run([API_CHECK, blob, str(d)], timeout=300)
    lines = out.strip().splitlines()
    assert lines[-1].startswith("ok"), out

    def f32(name, shape):
        return np.fromfile(d / name, np.float32).reshape(shape)

    for mode, tag in [(FLOAT, "float"), (FIXED, "fixed"), (INT8, "int8")]:
        want = oracle.bitlinear(x, nw, wq, scale, 1e-6, mode)
        assert_bitexact(f32(f"bl_{tag}.f32", (rows, N)), want["out"], f"bitlinear {tag}")
    want_fixed = oracle.bitlinear(x, nw, wq, scale, 1e-6, FIXED)["out"]
    assert_bitexact(f32("bl_fixed_cpube.f32", (rows, N)), want_fixed, "bitlinear through a CPU TernaryBackend")
    assert_bitexact(f32("bl_fixed_hipbe.f32", (rows, N)), want_fixed, "bitlinear through HipTernaryBackend")
    assert_bitexact(f32("bl_norm.f32", (rows, K)), oracle.rmsnorm(x, nw, 1e-6), "bitlinear norm_out")
    codes = np.fromfile(d / "hipbe_codes.i32", np.int32).reshape(rows, K)
    acc = np.fromfile(d / "hipbe_acc.i32", np.int32).reshape(rows, N)
    np.testing.assert_array_equal(acc, codes.astype(np.int64) @ wq.T.astype(np.int64))
    # one host buffer refilled with other weights: the second call uses the new weights
    w2 = np.fromfile(d / "hipbe_reuse_w2.i8", np.int8).reshape(N, K)
    assert not np.array_equal(w2, wq)
    np.testing.assert_array_equal(np.fromfile(d / "hipbe_reuse_acc1.i32", np.int32).reshape(rows, N),
                                  codes.astype(np.int64) @ wq.T.astype(np.int64))
    np.testing.assert_array_equal(np.fromfile(d / "hipbe_reuse_acc2.i32", np.int32).reshape(rows, N),
                                  codes.astype(np.int64) @ w2.T.astype(np.int64))
    # the host operator functions' projection cache follows a refilled buffer: weights (updated
    # in place), then norm weight and scale (the projection replaced)
    nw2 = np.fromfile(d / "bl_refill_nw2.f32", np.float32)
    for i, (w_, n_, s_) in enumerate([(wq, nw, scale), (w2, nw, scale), (w2, nw2, scale),
                                      (w2, nw2, float(np.float32(2.0 * scale)))]):
        assert_bitexact(f32(f"bl_refill{i}.f32", (rows, N)), oracle.bitlinear(x, n_, w_, s_, 1e-6, FIXED)["out"],
                        f"bitlinear on a refilled buffer, step {i}")
    cl = f32("cluster_cpube.f32", (3, rows, N))
    for j, s in enumerate((scale, 2.0 * scale, 0.5 * scale)):
        assert_bitexact(cl[j], oracle.bitlinear(x, nw, wq, float(np.float32(s)), 1e-6, FIXED)["out"],
                        f"bitlinear_cluster through a CPU TernaryBackend, projection {j}")
    assert_bitexact(f32("rmsnorm.f32", (rows, K)), oracle.rmsnorm(x, nw, 1e-6), "rmsnorm")
    assert_bitexact(f32("swishgate.f32", (rows, K)), oracle.rmsnorm_swishgate(x, o2, nw, 1e-6), "swishgate")
    assert_bitexact(f32("swiglu.f32", (rows, K)), oracle.swiglu(x, o2), "swiglu")
    st = np.full(K, 0.5, np.float32)
    want_out, want_st = oracle.hgrn_scan(x, fg, st)
    assert_bitexact(f32("scan.f32", (rows, K)), want_out, "hgrn_scan")
    assert_bitexact(np.fromfile(d / "scan_state.f32", np.float32), want_st, "hgrn_scan state")

    for mode, tag in [(FLOAT, "float"), (FIXED, "fixed")]:
        rm = ref.model(blob, mode)
        serve = _streams(d / f"serve_{tag}.txt")
        want = rm.generate_serve(prompts, 8)
        for g, w in zip(serve, want):
            np.testing.assert_array_equal(g, w)
        cb = _streams(d / f"serve_{tag}_cb.txt")
        for b, p in enumerate(prompts):
            np.testing.assert_array_equal(cb[b], serve[b][len(p):])
        want = rm.generate_serve(prompts, 8, temperature=0.8, top_k=40, seed=7)
        for g, w in zip(_streams(d / f"serve_{tag}_sampled.txt"), want):
            np.testing.assert_array_equal(g, w)
        np.testing.assert_array_equal(_streams(d / f"gen_{tag}_sampled.txt")[0],
                                      rm.generate(prompts[0], 24, temperature=0.8, top_k=40, seed=7))
        np.testing.assert_array_equal(_streams(d / f"gen_{tag}_sampled_full.txt")[0],
                                      rm.generate(prompts[0], 12, temperature=1.3, seed=11))
        g, gcb = _streams(d / f"gen_{tag}.txt")
        np.testing.assert_array_equal(g, rm.generate(prompts[0], 10))
        np.testing.assert_array_equal(gcb, g[len(prompts[0]):])
        rm.close()

    # Model::set_backend with backends that are not this engine's: every FixedQ510
    # projection's integer matmul on the host backend, results equal to the reference Model
    rm = ref.model(blob, FIXED)
    want_gen = rm.generate(prompts[0], 10)
    np.testing.assert_array_equal(_streams(d / "be_cpu_gen.txt")[0], want_gen)
    for g, w in zip(_streams(d / "be_cpu_serve.txt"), rm.generate_serve(prompts, 6)):
        np.testing.assert_array_equal(g, w)
    np.testing.assert_array_equal(_streams(d / "be_cpu_gen_sampled.txt")[0],
                                  rm.generate(prompts[0], 12, temperature=0.8, top_k=40, seed=7))
    want_lg = rm.forward(prompts[0])
    assert_bitexact(np.fromfile(d / "be_cpu_forward.f32", np.float32).reshape(want_lg.shape), want_lg,
                    "forward logits through a CPU TernaryBackend")
    rm.close()
    np.testing.assert_array_equal(_streams(d / "be_chunk_gen.txt")[0], want_gen)
    np.testing.assert_array_equal(_streams(d / "be_none_gen.txt")[0], want_gen)
    chk = next(ln for ln in lines if ln.startswith("chunked backend:"))
    counts = dict(kv.split("=") for kv in chk.split(":")[1].split())
    assert int(counts["calls"]) > 0 and int(counts["seq"]) > 0 and int(counts["lm_head_ids"]) > 0, chk
    assert counts["bad_ids"] == "0", chk
    assert "throwing backend: error propagated" in lines, out
