"""Shared fixtures. GPU tests carry @pytest.mark.gpu; the rest run on the CPU."""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def _ensure_oracle():
    so = os.path.join(ROOT, "oracle", "_build", "libmmf_oracle.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True, stdout=subprocess.DEVNULL)
    return so


@pytest.fixture(scope="session")
def oracle():
    _ensure_oracle()
    from oracle.oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    """The reference compiled from its own sources, if it was built here."""
    from oracle.oracle import REF_SO, Ref
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref not built (needs the reference sources at build time)")
    return Ref()


def _mkblob_bin():
    from matmulfreellmcpu_amd import MKBLOB
    if not os.path.exists(MKBLOB):
        subprocess.run(["make", "-C", os.path.join(ROOT, "matmulfreellmcpu_amd"), "_lib/mmfree-mkblob"],
                       check=True, stdout=subprocess.DEVNULL)
    return MKBLOB


@pytest.fixture(scope="session")
def blobs(tmp_path_factory):
    """Seeded synthetic blobs: name -> path. Random norm weights and lower bounds on the
    small shapes so that a misplaced weight or bound changes the result."""
    _mkblob_bin()
    from matmulfreellmcpu_amd import make_blob
    d = tmp_path_factory.mktemp("blobs")
    out = {}

    def get(name):
        if name in out:
            return out[name]
        p = str(d / f"{name}.mmfree")
        if name == "tiny":
            make_blob(p, preset="tiny", seed=7, random_norms=True, random_lb=True)
        elif name == "tiny_nolb":
            make_blob(p, preset="tiny", seed=8, random_norms=True, lower_bound=False)
        elif name == "small":
            make_blob(p, vocab=4096, hidden=256, layers=4, inter=704, seed=11, random_norms=True, random_lb=True)
        elif name == "wide":  # MLP gate matrix of 48 column tiles: the K-group GEMM at <= 64 rows
            make_blob(p, vocab=1024, hidden=1024, layers=2, inter=3072, seed=21, random_norms=True, random_lb=True)
        elif name == "tall":  # long prompts: 32 x 64 float matrix-core tiles in every GEMM kind
            make_blob(p, vocab=256, hidden=768, layers=1, inter=528, seed=31, random_norms=True, random_lb=True)
        elif name == "odd":  # hidden not a multiple of 8 or 16 (tails everywhere)
            make_blob(p, vocab=1000, hidden=100, layers=2, inter=208, seed=13, random_norms=True, random_lb=True)
        elif name == "s0":
            make_blob(p, preset="s0", seed=1234)
        elif name == "h2048":  # the 1.3B widths (hidden 2048, intermediate 5632, vocab 32000), 2 layers
            make_blob(p, vocab=32000, hidden=2048, layers=2, inter=5632, seed=41, random_norms=True, random_lb=True)
        elif name == "h2560":  # the 2.7B widths (hidden 2560, intermediate 6912, vocab 32000), 2 layers
            make_blob(p, vocab=32000, hidden=2560, layers=2, inter=6912, seed=43, random_norms=True, random_lb=True)
        else:
            raise KeyError(name)
        out[name] = p
        return p

    return get


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bitexact(a, b, what=""):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    assert a.shape == b.shape, f"{what}: shape {a.shape} vs {b.shape}"
    bad = bits(a) != bits(b)
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {int(bad.sum())} of {a.size} differ; first {idx.tolist()}: "
                             f"{a[tuple(idx[0])]!r} vs {b[tuple(idx[0])]!r}")
