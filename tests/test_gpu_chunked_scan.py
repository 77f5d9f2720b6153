"""The chunked parallel scan of float-mode prefills (mmf_model_set_scan(ctx, 1)).

It rounds differently from the reference's time-ordered recurrence, so these tests use the
float-mode tolerance instead of bit equality: identical greedy tokens, and logits within
1e-3 x max|logit| of the oracle (the CPU restatement of the reference). The default, the
time-ordered scan, stays bit-exact (every other float test).
"""
import numpy as np
import pytest

from conftest import assert_bitexact
from matmulfreellmcpu_amd import FLOAT

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3  # of max |logit|


def _close_logits(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.max(np.abs(got - want))
    scale = np.max(np.abs(want))
    assert err <= LOGIT_TOL * scale, f"{what}: max |err| {err:.3e} > {LOGIT_TOL} x {scale:.3e}"
    return err / scale


@pytest.mark.parametrize("n", [150, 600])
def test_chunked_forward_within_tolerance(blobs, oracle, n):
    """Full forward (every position's logits) on hidden 1024 with 150 and 600 tokens: whole
    and partial chunks, the lower bounds of layer 1. The result also differs from the exact
    scan somewhere, or the chunked path did not run."""
    from matmulfreellmcpu_amd import Engine, read_blob
    print(f"chunked forward n={n}", flush=True)
    blob = read_blob(blobs("wide"))
    ids = np.random.default_rng(n).integers(3, blob.config.vocab_size, n)
    want = oracle.model(blob).forward(ids, FLOAT)
    e = Engine(0)
    e.load_blob(blob, FLOAT)
    exact = e.forward(ids)
    assert_bitexact(exact, want, "time-ordered scan (default)")
    e.set_scan(True)
    got = e.forward(ids)
    rel = _close_logits(got, want, "chunked forward logits")
    # the greedy token of every position whose top two logits are further apart than twice
    # the largest logit difference (closer ones may legitimately swap)
    top2 = np.sort(want, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * np.max(np.abs(got - want))
    assert clear.sum() > 0.9 * n
    assert np.array_equal(np.argmax(got, axis=-1)[clear], np.argmax(want, axis=-1)[clear]), "argmax per position"
    assert rel > 0.0, "chunked scan gave the exact scan's logits: it did not run"
    e.set_scan(False)
    assert_bitexact(e.forward(ids), want, "time-ordered scan after switching back")
    e.close()


def test_chunked_generate_same_tokens(blobs, oracle):
    """B=1 greedy generate after a 200-token prefill on hidden 256 (4 layers): the same id
    stream as the reference and a recurrent state within 1e-4 relative."""
    from matmulfreellmcpu_amd import Engine, read_blob
    print("chunked generate", flush=True)
    blob = read_blob(blobs("small"))
    ids = np.random.default_rng(5).integers(3, blob.config.vocab_size, 200)
    want, wst = oracle.model(blob).generate(ids, 24, FLOAT, want_state=True)
    e = Engine(0)
    e.load_blob(blob, FLOAT)
    e.set_scan(True)
    got = e.generate(ids, 24)
    st = e.state()[:, 0, :]
    e.close()
    assert np.array_equal(got, want), f"ids {got.tolist()} != {want.tolist()}"
    d = np.max(np.abs(st.astype(np.float64) - wst)) / max(np.max(np.abs(wst)), 1e-30)
    assert d <= 1e-4, f"state relative difference {d:.3e}"


def test_set_scan_rejects_other_values(blobs):
    from matmulfreellmcpu_amd import Engine
    e = Engine(0)
    e.load_blob(blobs("tiny"), FLOAT)
    assert e.lib.mmf_model_set_scan(e.h, 2) == 1  # MMF_ERR_ARG
    e.close()
