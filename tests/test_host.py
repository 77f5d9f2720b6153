"""Host-side checks that need no GPU: the C ABI library loads and exports what
include/mmfree_hip.h declares, fails cleanly without a device, and the MMFREE1 blob reader and
the seeded blob generator behave as the reference's format requires."""
import ctypes as C
import hashlib
import json
import os
import re
import struct
import subprocess

import numpy as np
import pytest

import conftest

ROOT = conftest.ROOT
HEADER = os.path.join(ROOT, "include", "mmfree_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mmf_[a-z0-9_]+)\s*\(", text)) - {"mmf_token_cb"})


def test_library_exports_every_declared_symbol():
    from matmulfreellmcpu_amd import LIB_PATH
    lib = C.CDLL(LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 30
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, f"declared in mmfree_hip.h but not exported: {missing}"


def test_create_without_device_reports_nodev():
    """No GPU in this container: mmf_create must fail with MMF_ERR_NODEV, not crash."""
    import torch  # noqa: F401  (same process state as the other tests)
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from matmulfreellmcpu_amd import Engine, MmfError, load_library
    lib = load_library()
    h = C.c_void_p()
    assert lib.mmf_create(C.byref(h), 0) == 4
    assert b"device" in lib.mmf_last_error(None)
    with pytest.raises(MmfError):
        Engine(0)
    assert lib.mmf_sync(None) == 1  # MMF_ERR_ARG on a null context


def _write_blob(path, header, data_len, magic=b"MMFREE1\n"):
    hb = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(magic + struct.pack("<Q", len(hb)) + hb)
        f.write(b"\0" * ((-(16 + len(hb))) % 64))
        f.write(b"\0" * data_len)


def test_blob_reader_validates(tmp_path):
    from matmulfreellmcpu_amd import read_blob
    ok = {"config": {"vocab_size": 4, "hidden_size": 8}, "tensors": {
        "a": {"dtype": "f32", "shape": [2, 4], "offset": 0, "nbytes": 32}}}
    p = str(tmp_path / "ok.mmfree")
    _write_blob(p, ok, 64)
    b = read_blob(p)
    assert b.config.vocab_size == 4 and b.config.hidden_size == 8 and b.config.num_hidden_layers == 24
    assert b.get("a").shape == (2, 4)
    with pytest.raises(KeyError):
        b.get("missing")
    bad = str(tmp_path / "bad.mmfree")
    _write_blob(bad, ok, 64, magic=b"MMFREE2\n")
    with pytest.raises(ValueError, match="magic"):
        read_blob(bad)
    past = dict(ok, tensors={"a": {"dtype": "f32", "shape": [2, 4], "offset": 64, "nbytes": 32}})
    _write_blob(bad, past, 64)
    with pytest.raises(ValueError, match="does not fit"):
        read_blob(bad)
    wrongdt = dict(ok, tensors={"a": {"dtype": "f16", "shape": [2], "offset": 0, "nbytes": 4}})
    _write_blob(bad, wrongdt, 64)
    with pytest.raises(ValueError, match="dtype"):
        read_blob(bad)


def test_cxx_weights_reject_overflowing_shapes(tmp_path):
    """The C++ Weights loader (through mmfree-cli, which opens the blob before any device
    work) refuses shapes whose byte size wraps around 64 bits, and offsets past the end."""
    cli = os.path.join(ROOT, "matmulfreellmcpu_amd", "_lib", "mmfree-cli")
    if not os.path.exists(cli):
        pytest.skip("mmfree-cli not built")
    cases = {
        "wrap": {"dtype": "f32", "shape": [2 ** 33, 2 ** 31], "offset": 0, "nbytes": 0},
        "wrap3": {"dtype": "i8", "shape": [2 ** 32, 2 ** 16, 2 ** 16], "offset": 0},
        "offset": {"dtype": "f32", "shape": [2], "offset": 2 ** 52, "nbytes": 8},
    }
    for name, entry in cases.items():
        p = str(tmp_path / f"{name}.mmfree")
        _write_blob(p, {"config": {"vocab_size": 4, "hidden_size": 8}, "tensors": {"a": entry}}, 64)
        r = subprocess.run([cli, "--blob", p, "--ids", "1,2", "--gen", "1"], capture_output=True, text=True,
                           timeout=60)
        assert r.returncode == 1 and "does not fit the file" in r.stderr, (name, r.returncode, r.stderr)


def test_generator_is_deterministic_and_follows_the_recipe(tmp_path):
    from matmulfreellmcpu_amd import make_blob, read_blob
    conftest._mkblob_bin()
    a = make_blob(str(tmp_path / "a.mmfree"), preset="tiny", seed=5)
    b = make_blob(str(tmp_path / "b.mmfree"), preset="tiny", seed=5)
    c = make_blob(str(tmp_path / "c.mmfree"), preset="tiny", seed=6)
    h = [hashlib.sha256(open(x, "rb").read()).hexdigest() for x in (a, b, c)]
    assert h[0] == h[1] != h[2]
    blob = read_blob(a)
    cfg = blob.config
    names = ["model.embeddings", "model.norm.w", "lm_head.wq", "lm_head.scale_w", "lm_head.normw", "lower_bounds"]
    assert list(blob.tensors)[:6] == names  # provision.py:101-111 order
    wq = np.asarray(blob.get("model.layers.0.gate_proj.wq"))
    assert wq.shape == (2 * cfg.intermediate_size, cfg.hidden_size)
    assert set(np.unique(wq)) <= {-1, 0, 1}
    zeros = float((wq == 0).mean())
    assert 0.25 < zeros < 0.37  # N(0, s) ternarised at 0.5 * mean|W|: ~31% zeros
    lb = np.asarray(blob.get("lower_bounds"))
    L = cfg.num_hidden_layers
    np.testing.assert_allclose(lb[:, 0], np.arange(L) / L, atol=1e-6)  # raw zeros: lb[l] = l/L
    assert np.all(np.asarray(blob.get("model.norm.w")) == 1.0)
    emb = np.asarray(blob.get("model.embeddings"))
    assert abs(float(emb.std()) - 0.02) < 0.002
