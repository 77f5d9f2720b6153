#!/usr/bin/env python3
"""Decode throughput of the HGRN-Bit engine on one MI355X.

Headline (`value`): greedy decode tok/s at batch 1 on the 370M shape in float mode -- the
reference CLI's own benchmark (mmfree-cli --bench: 16-token prompt, greedy, decode tok/s),
on a seeded synthetic blob of that architecture. A step is one decode token: W untimed
steps, then exactly K timed steps (HIP events on the engine's stream, synchronised before
and after). The 1.3B and 2.7B shapes are reported beside it (`decode_tok_s`).

roofline: the decode kernel with the most time per token, its algorithmic bytes per launch
(2-bit packed weights + the fp32 vectors it must read and write once) over its average
launch duration, measured with an event pair around each launch (a child process with HIP
graphs off, MMF_GRAPH=0: `bench.py --roofline-leg`, the command the committed rocprofv3
summary traces); peak = 8 TB/s HBM. `traffic` (HBM bytes per launch from the calibrated
FETCH_SIZE/WRITE_SIZE runs in profiles/pmc_traffic.json) is written only while the digest of
the decode kernel sources recorded there matches the sources in this tree.

cpu_baseline: the reference engine compiled from its own sources (oracle/_ref/mmfree-cli,
built by oracle/Makefile) timed on this host's cores with its own --bench harness on the
same blob and prompt, on one socket's physical cores (OMP_PROC_BIND=close, one place per
core; `all_cpus`: every cpu this process may use); its greedy id stream is also compared
with the GPU's at every shape and mode (`parity`). `cpu_baselines` holds the same reference
beside the other workloads, each entry naming what was timed: the op sweep's integer matmul
(CpuBackend), the 1.3B prefill of 2048 tokens and decode of 256 (in full, as the reference's
own --bench harness runs it), and two lockstep serving steps per serving configuration.

Beside the headline (all on seeded synthetic weights of the named shapes):
  op_sweep  BitLinear with int8-absmax activations: x ~N(0,1) [M, K], M in {1, 16, 256,
            2048}, (K, N) in {(1024,1024), (1024,5632), (2816,1024), (2048,11264),
            (5632,2048)}; microseconds per call (RMSNorm + quantisation + ternary GEMM)
            with 20 calls back to back in one HIP graph (prologue_us / gemm_us: event
            pair around each launch), algorithmic bytes N*K/4 + 4MK + 4MN + 4K against
            8 TB/s, ops 2MNK against the 5.0 POP/s int8 peak.
  prefill   1.3B shape, 2048-token prompt, time to the first token (all layers + final
            norm, lm_head, argmax) per mode; per-GEMM microseconds and TOP/s (event pair
            around every launch); FixedQ510 runs two int8 passes (hi/lo code planes);
            float also with the opt-in chunked parallel scan (`chunked_scan`).
  serve     batched decode of independent streams (2.7B x 64 streams x 128-token prompts,
            float and FixedQ510; 1.3B x 32 x 512, FixedQ510): prompts prefilled together,
            then lockstep decode steps timed on the host around each step; weight bytes
            per step against 8 TB/s; `kinds_per_step`: microseconds per step in each
            launch kind and its weight GB/s (the step launched kernel by kernel with an
            event pair around every launch).
  decode_tok_s_fixed / kernels_fixed: the batch-1 decode in FixedQ510 (the reference CLI's
            default mode) at the three shapes.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import re
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s (B=1) 370M/1.3B/2.7B; BitLinear GB/s & % roofline, 1 GPU"
HBM_PEAK_GBS = 8000.0
SHAPES = {"370M": "s0", "1.3B": "s2", "2.7B": "s3"}
DIMS = {"s0": (32000, 1024, 24, 2816), "s2": (32000, 2048, 24, 5632), "s3": (32000, 2560, 32, 6912)}
KINDS = ("ifg", "o", "gate", "down", "lm")
MODE_NAMES = {0: "float", 1: "fixed"}
# the sources of the batch-1 decode kernels; profiles/pmc_traffic.json records their digest
DECODE_SOURCES = ("matmulfreellmcpu_amd/csrc/mmf_decode.hip", "matmulfreellmcpu_amd/csrc/mmf_device.hpp",
                  "matmulfreellmcpu_amd/csrc/mmf_internal.hpp")


def decode_sources_digest():
    h = hashlib.sha256()
    for p in DECODE_SOURCES:
        with open(os.path.join(ROOT, p), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_bytes(V, H, L, I):
    """Algorithmic HBM bytes per launch of each decode kernel: packed ternary weights
    (N*K/4) plus every fp32 vector read or written once (inputs, norm weights, state,
    outputs). Launches per token: L of each layer kind, one lm_head."""
    return {
        "ifg": 3 * H * H / 4 + 4 * (H + H + 3 * H + H + H) + 4 * 3 * H,  # h, attn_norm, 3 normw, lb, state | state, recur, g
        "o": H * H / 4 + 4 * (3 * H + 2 * H) + 4 * H,                    # g, recur, h, g_norm, normw | resid
        "gate": 2 * I * H / 4 + 4 * 3 * H + 4 * I,                       # resid, mlp_norm, normw | z
        "down": I * H / 4 + 4 * (2 * I + H) + 4 * H,                     # z, normw, resid | h
        "lm": V * H / 4 + 4 * 3 * H,                                     # h, norm, normw
    }, {"ifg": L, "o": L, "gate": L, "down": L, "lm": 1}


def blob_path(d, preset):
    from matmulfreellmcpu_amd import make_blob
    p = os.path.join(d, f"{preset}.mmfree")
    if not os.path.exists(p):
        t = time.time()
        make_blob(p, preset=preset, seed=1234)
        log(f"[bench] wrote {p} in {time.time() - t:.1f}s")
    return p


def roofline_leg(blob_dir, reps):
    """370M float decode, every launch between its own event pair (run with MMF_GRAPH=0, so no
    HIP graph): prints the microseconds per launch of each kind."""
    from matmulfreellmcpu_amd import FLOAT, Engine
    e = Engine(0)
    e.load_blob(blob_path(blob_dir, "s0"), FLOAT)
    e.generate(np.random.default_rng(1234).integers(3, 32000, 16), 8)
    _, kind_us = e.time_decode(warmup=4, reps=reps)
    e.close()
    print(json.dumps({k: round(v, 3) for k, v in kind_us.items()}))


def measure(eng, preset, steps, warmup):
    V, H, L, I = DIMS[preset]
    step_us, kind_us = eng.time_decode(warmup=warmup, reps=steps)
    nbytes, nlaunch = kernel_bytes(V, H, L, I)
    kernels = {}
    for k in KINDS:
        us = kind_us[k]
        kernels[k] = {"us_per_launch": round(us, 3), "launches_per_token": nlaunch[k],
                      "bytes_per_launch": int(nbytes[k]), "GBps": round(nbytes[k] / us / 1e3, 1),
                      "frac": round(nbytes[k] / us / 1e3 / HBM_PEAK_GBS, 4)}
    tok_bytes = sum(nbytes[k] * nlaunch[k] for k in KINDS)
    return step_us, kernels, tok_bytes


INT8_PEAK_TOPS = 5000.0
SWEEP_KN = [(1024, 1024), (1024, 5632), (2816, 1024), (2048, 11264), (5632, 2048)]
SWEEP_M = [1, 16, 256, 2048]


def measure_op_sweep(reps):
    """BitLinear (int8 absmax) over the op-sweep shapes on device-resident inputs."""
    import ctypes as C
    from matmulfreellmcpu_amd import INT8_ABSMAX, Engine
    e = Engine(0)
    rng = np.random.default_rng(2024)
    out = []

    def dev(nbytes, arr=None):
        p = C.c_void_p()
        e._chk(e.lib.mmf_malloc(e.h, C.byref(p), nbytes))
        if arr is not None:
            e._chk(e.lib.mmf_upload(e.h, p, arr.ctypes.data_as(C.c_void_p), nbytes))
        return p.value

    for K, N in SWEEP_KN:
        latent = rng.standard_normal((N, K)).astype(np.float32) * 0.02
        scale = np.float32(1.0) / np.float32(np.abs(latent).mean())
        wq = np.clip(np.rint(latent * scale), -1, 1).astype(np.int8)
        pid = e.register_proj(wq, float(scale), np.ones(K, np.float32))
        for M in SWEEP_M:
            x = rng.standard_normal((M, K)).astype(np.float32)
            dx, do = dev(x.nbytes, x), dev(M * N * 4)
            total, pro, gemm = e.time_bitlinear(pid, dx, do, M, mode=INT8_ABSMAX, warmup=3, reps=reps)
            nbytes = N * K / 4 + 4 * M * K + 4 * M * N + 4 * K
            ops = 2.0 * M * N * K
            bound = "mfma" if ops / nbytes > INT8_PEAK_TOPS * 1e12 / (HBM_PEAK_GBS * 1e9) else "hbm"
            out.append({"M": M, "K": K, "N": N, "us": round(total, 2), "prologue_us": round(pro, 2),
                        "gemm_us": round(gemm, 2), "GBps": round(nbytes / total / 1e3, 1),
                        "hbm_frac": round(nbytes / total / 1e3 / HBM_PEAK_GBS, 4),
                        "TOPS": round(ops / total / 1e6, 2), "mfma_frac": round(ops / total / 1e6 / INT8_PEAK_TOPS, 4),
                        "bound": bound})
            e.lib.mmf_free(e.h, dx)
            e.lib.mmf_free(e.h, do)
    e.close()
    return out


def vendor_int8_gemm(T, H, I, reps=20):
    """The vendor library's dense int8 GEMM (hipBLASLt through torch._int_mm) on the four
    projection shapes of one prefill layer: rows T, int8 activations times int8 weights
    (here ternary values stored as full int8), int32 out. Reported beside the prefill
    GEMMs as the rate a tuned library reaches at the same M, N, K."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(5)
    shapes = {"gemm_ifg": (H, 3 * H), "gemm_o": (H, H), "gemm_gate": (H, 2 * I), "gemm_down": (I, H)}
    out = {}
    for k, (K, N) in shapes.items():
        a = torch.randint(-127, 128, (T, K), dtype=torch.int8, device="cuda", generator=g)
        w = torch.randint(-1, 2, (N, K), dtype=torch.int8, device="cuda", generator=g).t()  # K x N, column-major
        torch._int_mm(a, w)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            torch._int_mm(a, w)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        out[k] = round(2.0 * T * K * N / us / 1e6, 1)
    return out


def measure_prefill(blob_dir, T=2048, modes=("fixed", "int8", "float")):
    from matmulfreellmcpu_amd import MODES, Engine
    V, H, L, I = DIMS["s2"]
    p = blob_path(blob_dir, "s2")
    ids = np.random.default_rng(77).integers(3, 32000, T)
    res = {}
    for name in modes:
        mode = MODES[name]
        e = Engine(0)
        e.load_blob(p, mode)
        total, kinds = e.time_prefill(ids, warmup=1, reps=3)
        chunked = None
        if name == "float":
            # the opt-in chunked parallel scan (within fp32 rounding of the reference, not equal)
            e.set_scan(True)
            ctotal, ckinds = e.time_prefill(ids, warmup=1, reps=3)
            e.set_scan(False)
            chunked = {"ms": round(ctotal / 1e3, 3), "mixer_ms": round(ckinds["mixer"] / 1e3, 3)}
        e.close()
        r = {"ms": round(total / 1e3, 3), "tok_s": round(T / total * 1e6, 1),
             "kinds_ms": {k: round(v / 1e3, 3) for k, v in kinds.items()}}
        if chunked:
            r["chunked_scan"] = chunked
        if name != "float":
            planes = 2 if name == "fixed" else 1
            ops = {"gemm_ifg": 2.0 * T * 3 * H * H * L, "gemm_o": 2.0 * T * H * H * L,
                   "gemm_gate": 2.0 * T * 2 * I * H * L, "gemm_down": 2.0 * T * H * I * L}
            r["gemm_TOPS"] = {k: round(ops[k] / kinds[k] / 1e6, 1) for k in ops}
            r["mfma_TOPS"] = {k: round(planes * ops[k] / kinds[k] / 1e6, 1) for k in ops}
            allops = sum(ops.values())
            alltime = sum(kinds[k] for k in ops)
            r["mfma_frac_all_gemms"] = round(planes * allops / alltime / 1e6 / INT8_PEAK_TOPS, 4)
        res[name] = r
        log(f"[bench] prefill 1.3B T={T} {name}: {r['ms']} ms ({r['tok_s']} tok/s)")
    # torch's bundled HIP runtime cannot open the device in a process where this library's
    # runtime already has it: the comparison runs in a child process that imports only torch
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-int8", f"{T},{H},{I}"],
                           capture_output=True, text=True, timeout=300, check=True)
        res["vendor_int8_gemm_TOPS"] = json.loads(r.stdout.strip().splitlines()[-1])
        log(f"[bench] hipBLASLt int8 GEMM at the same shapes (TOP/s): {res['vendor_int8_gemm_TOPS']}")
    except Exception as ex:  # a comparison line only; the prefill numbers stand without it
        log(f"[bench] vendor int8 GEMM comparison skipped: {ex}")
    return res


def serve_leg(blob_dir, cfgs):
    """Serving steps only, untimed (PRESET:MODE:B:T:STEPS per config): the program of the
    serving-step counter runs."""
    from matmulfreellmcpu_amd import MODES, Engine
    os.makedirs(blob_dir, exist_ok=True)
    for cfg in cfgs.split(","):
        preset, mode, B, T, steps = cfg.split(":")
        B, T, steps = int(B), int(T), int(steps)
        e = Engine(0)
        e.load_blob(blob_path(blob_dir, preset), MODES[mode])
        e.reset(B)
        cur = e.prefill_streams(np.random.default_rng(1).integers(3, 32000, (B, T)))
        for _ in range(steps):
            cur = e.step(cur)
        e.close()
        log(f"[bench] serve leg {cfg} done")


def measure_serve(blob_dir, preset, B, T, mode_name, steps):
    from matmulfreellmcpu_amd import MODES, Engine
    p = blob_path(blob_dir, preset)
    e = Engine(0)
    e.load_blob(p, MODES[mode_name])
    rng = np.random.default_rng(B * 1000 + T)
    prompts = rng.integers(3, 32000, (B, T))
    e.reset(B)
    t0 = time.perf_counter()
    cur = e.prefill_streams(prompts)
    t_pre = time.perf_counter() - t0
    for _ in range(2):
        cur = e.step(cur)
    t0 = time.perf_counter()
    for _ in range(steps):
        cur = e.step(cur)
    dt = time.perf_counter() - t0
    # per launch kind: the same step launched kernel by kernel, an event pair around each
    kinds = e.time_step_kinds(cur, warmup=1, reps=4)
    e.close()
    V, H, L, I = DIMS[preset]
    kbytes = {"gemm_ifg": L * 3 * H * H / 4, "gemm_o": L * H * H / 4, "gemm_gate": L * 2 * I * H / 4,
              "gemm_down": L * H * I / 4, "lm": V * H / 4}  # packed ternary weights per kind and step
    kind_r = {k: {"us": round(v, 1)} for k, v in kinds.items() if v > 0}
    for k, b in kbytes.items():
        if kinds.get(k, 0) > 0:
            kind_r[k]["weight_GBps"] = round(b / kinds[k] / 1e3, 1)
            kind_r[k]["hbm_frac"] = round(b / kinds[k] / 1e3 / HBM_PEAK_GBS, 4)
    wbytes = L * (4 * H * H + 3 * I * H) / 4 + V * H / 4  # packed ternary weights read per step
    ops = 2.0 * B * (L * (4 * H * H + 3 * I * H) + V * H)
    step_s = dt / steps
    r = {"streams": B, "prompt_tokens": T, "mode": mode_name, "steps_timed": steps,
         "ms_per_step": round(step_s * 1e3, 3), "decode_tok_s": round(B * steps / dt, 1),
         "prefill_s": round(t_pre, 3), "weight_GBps": round(wbytes / step_s / 1e9, 1),
         "hbm_frac": round(wbytes / step_s / 1e9 / HBM_PEAK_GBS, 4),
         "TOPS": round(ops / step_s / 1e12, 2), "kinds_per_step": kind_r}
    log(f"[bench] serve {preset} B={B} T={T} {mode_name}: {r['ms_per_step']} ms/step, {r['decode_tok_s']} tok/s")
    return r


# ---- CPU baselines: the reference engine compiled from its own sources (oracle/_ref) -------

REF_CLI = os.path.join(ROOT, "oracle", "_ref", "mmfree-cli")


def cpu_sets():
    """(cpus of one socket, one per physical core; every cpu this process may use): the
    socket is the one holding most of the allowed cpus."""
    cpus = sorted(os.sched_getaffinity(0))
    sockets = {}
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            pkg = int(open(base + "physical_package_id").read())
            core = int(open(base + "core_id").read())
        except (OSError, ValueError):
            pkg, core = 0, c
        sockets.setdefault(pkg, {}).setdefault(core, c)
    pkg = max(sockets, key=lambda p: len(sockets[p]))
    return sorted(sockets[pkg].values()), cpus


def omp_env(cpus):
    """OpenMP settings for a CPU run on exactly `cpus`: one thread each, bound in order, threads
    spinning between parallel regions (the reference's many short regions start faster)."""
    places = ",".join("{%d}" % c for c in cpus)
    return dict(os.environ, OMP_NUM_THREADS=str(len(cpus)), OMP_PROC_BIND="close", OMP_PLACES=places,
                OMP_WAIT_POLICY="active")


def ref_cli_bench(blob, ids, gen, mode, env, reps=3, warmup=1):
    """The reference CLI's own --bench (bench.cpp:42-112): (avg prefill ms, avg decode tok/s, wall s)."""
    t = time.time()
    r = subprocess.run([REF_CLI, "--blob", blob, "--ids", ",".join(str(int(i)) for i in ids), "--bench", "--gen",
                        str(gen), "--warmup", str(warmup), "--reps", str(reps), "--mode", mode],
                       capture_output=True, text=True, env=env, check=True, timeout=600)
    wall = time.time() - t
    pre = re.search(r"avg prefill:\s+([0-9.]+) ms", r.stdout)
    dec = re.search(r"avg decode:\s+([0-9.]+) tok/s", r.stdout)
    return (float(pre.group(1)) if pre else None), (float(dec.group(1)) if dec else None), wall


def cpu_leg(job):
    """One CPU baseline job in this (child) process, whose OpenMP settings the parent set:
    prints one JSON line. Jobs run the reference compiled from its sources."""
    from oracle.oracle import FIXED, FLOAT, Ref
    kind, arg = job.split(":", 1) if ":" in job else (job, "")
    if kind == "op_sweep":  # CpuBackend::matmul_batch (ternary_backend.hpp:96-103) at every sweep shape
        ref = Ref()
        rng = np.random.default_rng(7)
        out = []
        for K, N in SWEEP_KN:
            wq = rng.integers(-1, 2, (N, K)).astype(np.int8)
            for M in SWEEP_M:
                x = rng.integers(-128, 128, (M, K)).astype(np.int32)
                ref.ternary_matmul(x, wq)  # first touch of the weights, thread pool up
                t = time.perf_counter()
                ref.ternary_matmul(x, wq)
                us = (time.perf_counter() - t) * 1e6
                nbytes = N * K / 4 + 4 * M * K + 4 * M * N + 4 * K
                out.append({"M": M, "K": K, "N": N, "us": round(us, 1), "GBps": round(nbytes / us / 1e3, 2),
                            "TOPS": round(2.0 * M * N * K / us / 1e6, 3)})
        print(json.dumps(out))
    elif kind == "serve":  # Model::generate_serve (hgrn_model.cpp:349-454): time per lockstep step
        blob, B, mode = arg.split(",")
        B = int(B)
        rm = Ref().model(blob, FIXED if mode == "fixed" else FLOAT)
        prompts = [[3 + (7 * b) % 31000] for b in range(B)]  # one-token prompts: prefill = one row per stream
        rm.generate_serve(prompts, 1)
        t = time.perf_counter()
        rm.generate_serve(prompts, 1)
        t1 = time.perf_counter() - t
        t = time.perf_counter()
        rm.generate_serve(prompts, 3)
        t3 = time.perf_counter() - t
        rm.close()
        step = max(t3 - t1, 1e-9) / 2
        print(json.dumps({"ms_per_step": round(step * 1e3, 1), "tok_s": round(B / step, 1)}))
    elif kind == "seam":  # the reference Model with HipTernaryBackend at its TernaryBackend seam
        import ctypes as C
        from oracle.oracle import Ref
        so = os.path.join(ROOT, "oracle", "_ref", "libmmfree_ref_hipbe.so")
        r = Ref(so)
        L = r.lib
        L.ref_model_ptr.restype = C.c_void_p
        L.ref_model_ptr.argtypes = [C.c_void_p]
        L.ref_model_weights.restype = C.c_void_p
        L.ref_model_weights.argtypes = [C.c_void_p]
        L.ref_hipbe_attach.restype = C.c_void_p
        L.ref_hipbe_attach.argtypes = [C.c_void_p, C.c_int]
        L.ref_hipbe_attach_registered.restype = C.c_void_p
        L.ref_hipbe_attach_registered.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
        L.ref_hipbe_detach.argtypes = [C.c_void_p, C.c_void_p]
        blob, n = arg.split(",")
        n = int(n)
        ids = np.random.default_rng(1234).integers(3, 32000, 16)

        def rate(m, gen):  # decode tok/s: (gen - 1) tokens over the time beyond a 1-token run
            m.generate(ids, 2)
            t = time.perf_counter()
            m.generate(ids, 1)
            t1 = time.perf_counter() - t
            t = time.perf_counter()
            out = m.generate(ids, gen)
            tn = time.perf_counter() - t
            return (gen - 1) / max(tn - t1, 1e-9), out

        res = {}
        m = r.model(blob, FIXED)
        cpu_rate, want = rate(m, n)
        res["cpu"] = round(cpu_rate, 1)
        for label, attach, gen in (("registered", "reg", n), ("proj_id_minus_1", "raw", max(8, n // 8))):
            mp = L.ref_model_ptr(m.h)
            be = (L.ref_hipbe_attach_registered(mp, L.ref_model_weights(m.h), 0) if attach == "reg"
                  else L.ref_hipbe_attach(mp, 0))
            if not be:
                raise SystemExit("attaching HipTernaryBackend failed")
            try:
                g, got = rate(m, gen)
            finally:
                L.ref_hipbe_detach(mp, be)
            res[label] = {"decode_tok_s": round(g, 1), "tokens": gen,
                          "ids_identical": bool(np.array_equal(got, want[:got.size]))}
        m.close()
        print(json.dumps(res))
    else:
        raise SystemExit(f"unknown cpu job {job}")


def run_cpu_leg(job, cpus, timeout=600):
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-leg", job], capture_output=True, text=True,
                       env=omp_env(cpus), check=True, timeout=timeout)
    return json.loads(r.stdout.strip().splitlines()[-1])


def ref_cli_ids(blob, ids, gen, mode, env):
    """Greedy ids from the reference CLI (prompt and generated tokens, as --print-ids prints them)."""
    r = subprocess.run([REF_CLI, "--blob", blob, "--ids", ",".join(str(int(i)) for i in ids), "--gen", str(gen),
                        "--mode", mode, "--print-ids"], capture_output=True, text=True, env=env, check=True,
                       timeout=600)
    return np.array([int(t) for t in r.stdout.split()], np.int64)


def cpu_baselines(blob_dir, ids, gen, gpu_ids):
    """The reference engine on this host's cores beside every workload: one socket's
    physical cores (OMP_PROC_BIND=close, one place per core), and for the headline also every
    allowed cpu. Each dict says what was timed. gpu_ids[(shape, mode)]: the GPU's greedy ids
    for the 16-token prompt, compared with the reference CLI's."""
    if not os.path.exists(REF_CLI):
        return None, None, {}, None
    sock, allc = cpu_sets()
    env_s, env_a = omp_env(sock), omp_env(allc)
    res = {}
    parity = {"against": "reference mmfree-cli (oracle/_ref), 16-token prompt, greedy", "tokens": gen, "shapes": {}}
    for (name, mode), got in sorted(gpu_ids.items()):
        want = ref_cli_ids(blob_path(blob_dir, SHAPES[name]), ids, gen, mode, env_s)
        parity["shapes"].setdefault(name, {})[mode] = bool(np.array_equal(want, got))
    parity["ids_identical"] = all(v for d in parity["shapes"].values() for v in d.values())
    log(f"[bench] parity with the reference CLI: {parity['shapes']}")
    # config 0: the reference CLI's --bench on the 370M blob, float, as the GPU headline
    blob0 = blob_path(blob_dir, "s0")
    _, tps, wall = ref_cli_bench(blob0, ids, gen, "float", env_s)
    _, tps_all, wall_all = ref_cli_bench(blob0, ids, gen, "float", env_a)
    head = {"value": tps, "unit": "tok/s", "cores": len(sock), "kind": "reference",
            "sample": f"370M float, 16-token prompt, {gen} greedy tokens: reference mmfree-cli --bench warmup 1 "
                      f"reps 3 ({wall:.1f}s wall) on one socket's {len(sock)} physical cores, OMP_PROC_BIND=close, "
                      "OMP_WAIT_POLICY=active",
            "all_cpus": {"value": tps_all, "cores": len(allc), "wall_s": round(wall_all, 1)}}
    log(f"[bench] cpu reference 370M float: {tps} tok/s on {len(sock)} cores, {tps_all} on {len(allc)} cpus")
    # config 2 in full: 1.3B, 2048-token prefill then 256 greedy tokens, float and fixed
    blob2 = blob_path(blob_dir, "s2")
    ids2k = np.random.default_rng(77).integers(3, 32000, 2048)
    c2 = {}
    for mode in ("float", "fixed"):
        pre_ms, dec, wall = ref_cli_bench(blob2, ids2k, 256, mode, env_s, reps=1, warmup=0)
        c2[mode] = {"prefill_ms": pre_ms, "prefill_tok_s": round(2048 / pre_ms * 1e3, 2) if pre_ms else None,
                    "decode_tok_s": dec, "wall_s": round(wall, 1)}
    res["prefill_decode_1.3B"] = {"kind": "reference", "cores": len(sock), "modes": c2,
                                  "sample": "1.3B, 2048-token prompt + 256 greedy tokens (configuration 2 in full), "
                                            "reference mmfree-cli --bench warmup 0 reps 1"}
    log(f"[bench] cpu reference 1.3B: {c2}")
    # config 1: the op sweep's integer matmul through the reference's CpuBackend
    res["op_sweep"] = {"kind": "reference", "cores": len(sock), "shapes": run_cpu_leg("op_sweep", sock),
                       "sample": "CpuBackend::matmul_batch on int8-range codes at every (M, K, N), one call each"}
    # the drop-in at the seam: the reference Model (FixedQ510, 370M) with its integer
    # projections through HipTernaryBackend, beside the same Model on the CPU
    try:
        seam = run_cpu_leg(f"seam:{blob_path(blob_dir, 's0')},64", sock)
        res["seam_370M_fixed"] = dict(seam, kind="reference", cores=len(sock),
                                      sample="reference Model::generate, 370M FixedQ510, 16-token prompt: decode "
                                             "tok/s on the CPU (CpuBackend) and with HipTernaryBackend, registered "
                                             "(tag registry of resident projections) and proj_id -1 (exact "
                                             "check of the weights at each call); ids compared with the CPU run")
        log(f"[bench] seam: {seam}")
    except Exception as ex:
        log(f"[bench] seam leg failed: {ex}")
    # configs 3 and 4: lockstep serving steps
    for key, preset, B, mode in (("serve_2.7B_x64_float", "s3", 64, "float"), ("serve_2.7B_x64_fixed", "s3", 64, "fixed"),
                                 ("serve_1.3B_x32_fixed", "s2", 32, "fixed")):
        r = run_cpu_leg(f"serve:{blob_path(blob_dir, preset)},{B},{mode}", sock)
        res[key] = dict(r, kind="reference", cores=len(sock),
                        sample=f"Model::generate_serve, {B} one-token prompts, 2 lockstep steps timed (3 new tokens "
                               "minus 1)")
        log(f"[bench] cpu reference {key}: {r}")
    return head, res, parity


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512, help="timed decode steps (tokens) on the headline shape")
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--shapes", default="370M,1.3B,2.7B")
    ap.add_argument("--blob-dir", default=os.environ.get("MMF_BLOB_DIR", "/tmp/mmf_bench_blobs"))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU reference baseline")
    ap.add_argument("--sections", default="decode,op_sweep,prefill,serve",
                    help="comma list of decode,op_sweep,prefill,serve (decode is always run)")
    ap.add_argument("--vendor-int8", default=None, metavar="T,H,I",
                    help="only time the vendor int8 GEMM on one prefill layer's shapes (child process)")
    ap.add_argument("--cpu-leg", default=None, help="run one CPU baseline job (child process)")
    ap.add_argument("--roofline-leg", action="store_true",
                    help="only the 370M float decode with an event pair around every launch (run with "
                         "MMF_GRAPH=0; child process of the roofline, and the command rocprofv3 traces)")
    ap.add_argument("--serve-leg", default=None, metavar="PRESET:MODE:B:T:STEPS[,...]",
                    help="only run serving steps (prefill B prompts of T tokens, then STEPS lockstep steps) "
                         "for each listed config, untimed: the program the serving counter runs profile")
    ap.add_argument("--skip-decode", action="store_true",
                    help="profiling runs of the other sections: no B=1 decode and no headline (the "
                         "printed line holds only the sections run)")
    ap.add_argument("--decode-modes", default="float,fixed",
                    help="comma list of float,fixed: the batch-1 decode modes timed (float always runs: it carries the headline)")
    args = ap.parse_args()
    if args.cpu_leg:
        cpu_leg(args.cpu_leg)
        return
    if args.roofline_leg:
        os.makedirs(args.blob_dir, exist_ok=True)
        roofline_leg(args.blob_dir, max(16, args.steps // 4))
        return
    if args.serve_leg:
        serve_leg(args.blob_dir, args.serve_leg)
        return
    if args.vendor_int8:
        T, H, I = (int(x) for x in args.vendor_int8.split(","))
        print(json.dumps(vendor_int8_gemm(T, H, I)))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the HGRN-Bit hot path here runs on a single MI355X and this "
              f"build has no multi-GPU path (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    os.makedirs(args.blob_dir, exist_ok=True)
    from matmulfreellmcpu_amd import FIXED_Q510, FLOAT, Engine

    eng = Engine(0)
    devname, cus = eng.device_info()
    log(f"[bench] device {devname}, {cus} CUs")
    peaks = eng.measure_peaks()
    log(f"[bench] measured ceilings: {peaks}")
    shapes = [s.strip() for s in args.shapes.split(",") if s.strip()]
    dm = {x.strip() for x in args.decode_modes.split(",")}
    decode_modes = {FLOAT: True, FIXED_Q510: "fixed" in dm}
    if "370M" not in shapes:
        shapes.insert(0, "370M")
    results = {}
    ids = np.random.default_rng(1234).integers(3, 32000, 16)
    gpu_ids = {}  # (shape, mode name) -> greedy ids of the 16-token prompt, 128 tokens
    fixed = {}
    for name in ([] if args.skip_decode else shapes):
        preset = SHAPES[name]
        p = blob_path(args.blob_dir, preset)
        for mode in [m for m in (FLOAT, FIXED_Q510) if decode_modes[m]]:
            t = time.time()
            eng.close()
            eng = Engine(0)
            eng.load_blob(p, mode)
            log(f"[bench] {name} mode {mode}: loaded + repacked in {time.time() - t:.1f}s")
            gpu_ids[(name, MODE_NAMES[mode])] = eng.generate(ids, 128)
            eng.generate(ids, 16)
            steps = args.steps if (name == "370M" and mode == FLOAT) else max(64, args.steps // 4)
            eng.sync()
            t0 = time.perf_counter()
            step_us, kernels, tok_bytes = measure(eng, preset, steps, args.warmup)
            eng.sync()
            wall = time.perf_counter() - t0
            r = dict(step_us=step_us, kernels=kernels, tok_bytes=tok_bytes, steps=steps, wall=wall)
            if mode == FLOAT:
                results[name] = r
            else:
                fixed[name] = r
            log(f"[bench] {name} mode {mode}: {1e6 / step_us:.1f} tok/s ({step_us:.1f} us/token), "
                + ", ".join(f"{k} {v['us_per_launch']:.2f}us {v['GBps']:.0f}GB/s" for k, v in kernels.items()))
    eng.close()
    sections = {x.strip() for x in args.sections.split(",")}
    extra = {}
    if "op_sweep" in sections:
        extra["op_sweep"] = measure_op_sweep(reps=20)
    if "prefill" in sections:
        extra["prefill"] = measure_prefill(args.blob_dir)
    if "serve" in sections:
        extra["serve"] = [measure_serve(args.blob_dir, "s3", 64, 128, "float", 32),
                          measure_serve(args.blob_dir, "s3", 64, 128, "fixed", 32),
                          measure_serve(args.blob_dir, "s2", 32, 512, "fixed", 32)]

    if args.skip_decode:
        print(json.dumps({"metric": METRIC, "value": None, "sections": sorted(sections), **extra}), flush=True)
        return
    head = results["370M"]
    value = 1e6 / head["step_us"]
    kern = head["kernels"]
    dom = max(KINDS, key=lambda k: kern[k]["us_per_launch"] * kern[k]["launches_per_token"])
    # that kind's average launch from events recorded at each launch's own start and end
    # (hipExtLaunchKernelGGL), graphs off (a child process: MMF_GRAPH is read once per process)
    leg_us = None
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--roofline-leg", "--steps", str(args.steps),
                            "--blob-dir", args.blob_dir], capture_output=True, text=True, timeout=300, check=True,
                           env=dict(os.environ, MMF_GRAPH="0"))
        leg_us = json.loads(r.stdout.strip().splitlines()[-1])
    except Exception as ex:  # the graph-replay figure stands in, and the line says so
        log(f"[bench] roofline leg failed: {ex}")
    us = leg_us[dom] if leg_us else kern[dom]["us_per_launch"]
    achieved = round(kern[dom]["bytes_per_launch"] / us / 1e3, 1)
    # HBM bytes per launch of that kernel from the committed PMC summary (FETCH_SIZE and
    # WRITE_SIZE runs, calibrated on a copy kernel of known size), only while it describes the
    # kernels of this tree (the digest of their sources recorded with it)
    traffic, traffic_kernel = None, None
    try:
        with open(os.path.join(ROOT, "profiles", "pmc_traffic.json")) as f:
            pmc = json.load(f)
        if pmc.get("sources_sha256") == decode_sources_digest():
            traffic = pmc["kernels"][dom]["traffic_bytes"]
            traffic_kernel = pmc["kernels"][dom]["kernel"]
        else:
            log("[bench] profiles/pmc_traffic.json describes other decode sources: traffic left null")
    except (OSError, KeyError, ValueError):
        pass
    roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": f"370M float {dom}" + (f" ({traffic_kernel})" if traffic_kernel else ""),
                "bytes_per_launch": kern[dom]["bytes_per_launch"], "us_per_launch": us,
                "timing": "the kernel's own start and end events (hipExtLaunchKernelGGL), HIP graphs off" if leg_us
                          else "graph replay (the event leg failed)",
                "us_per_launch_graph_replay": kern[dom]["us_per_launch"]}

    cpu = None
    parity = None
    cpu_configs = {}
    if not args.no_cpu:
        cpu, cpu_configs, parity = cpu_baselines(args.blob_dir, ids, 128, gpu_ids)

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(head["step_us"] / 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded ternary weights ~N(0,0.02) -> {-1,0,1}, embeddings ~N(0,0.02), norms 1)",
        "config": {"workload": "HGRN-Bit 370M (H1024 I2816 L24 V32000) greedy decode, batch 1, float mode, "
                               "16-token random prompt", "batch": 1, "prompt_tokens": 16, "mode": "float"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "decode_tok_s": {n: round(1e6 / r["step_us"], 1) for n, r in results.items()},
        "step_GBps": {n: round(r["tok_bytes"] / r["step_us"] / 1e3, 1) for n, r in results.items()},
        "kernels": {n: r["kernels"] for n, r in results.items()},
        "decode_tok_s_fixed": {n: round(1e6 / r["step_us"], 1) for n, r in fixed.items()},
        "kernels_fixed": {n: r["kernels"] for n, r in fixed.items()},
        "cpu_baselines": cpu_configs,
        "parity": parity,
        "device": f"{devname}, {cus} CUs",
        "measured_ceilings": peaks,
    }
    out.update(extra)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
