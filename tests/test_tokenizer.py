"""Tokenizer (the CLI's text path) against the reference tokenizer compiled from its own
sources (oracle/_ref, cpp/src/io/tokenizer.cpp), on synthetic tokenizer.mmtok files:
encode with and without BOS, decode with and without the special tokens, id for id and
byte for byte; plus the CLI paths that need no model (--decode-ids, --gen 0 --print-ids).
CPU only."""
import ctypes as C
import os
import random
import struct
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from tok_util import make_tokenizer, random_texts, write_mmtok

TOK_CHECK = os.path.join(ROOT, "tests", "cpp", "_build", "tok_check")
CLI = os.path.join(ROOT, "matmulfreellmcpu_amd", "_lib", "mmfree-cli")


def _need(p):
    if not os.path.exists(p):
        pytest.skip(f"{os.path.relpath(p, ROOT)} not built")


@pytest.fixture(scope="module")
def reflib():
    from oracle.oracle import REF_SO
    _need(REF_SO)
    L = C.CDLL(REF_SO)
    L.ref_tok_open.restype = C.c_void_p
    L.ref_tok_open.argtypes = [C.c_char_p]
    L.ref_tok_close.argtypes = [C.c_void_p]
    L.ref_tok_encode.restype = C.c_long
    L.ref_tok_encode.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t, C.c_int, C.POINTER(C.c_int64), C.c_size_t]
    L.ref_tok_decode.restype = C.c_long
    L.ref_tok_decode.argtypes = [C.c_void_p, C.POINTER(C.c_int64), C.c_size_t, C.c_int, C.c_char_p, C.c_size_t]
    return L


def ref_encode(L, h, text, bos):
    out = (C.c_int64 * (4 * len(text) + 8))()
    n = L.ref_tok_encode(h, text, len(text), int(bos), out, len(out))
    assert n <= len(out)
    return list(out[:n])


def ref_decode(L, h, ids, skip):
    arr = (C.c_int64 * max(len(ids), 1))(*ids)
    buf = C.create_string_buffer(16 * len(ids) + 16)
    n = L.ref_tok_decode(h, arr, len(ids), int(skip), buf, len(buf))
    assert n <= len(buf)
    return buf.raw[:n]


def ours(tok_path, texts, id_lists, tmp):
    req = bytearray()
    for t in texts:
        req += b"\x00" + struct.pack("<I", len(t)) + t
    for ids in id_lists:
        req += b"\x01" + struct.pack("<I", len(ids)) + np.asarray(ids, np.int64).tobytes()
    rq, rs = os.path.join(tmp, "req.bin"), os.path.join(tmp, "res.bin")
    open(rq, "wb").write(bytes(req))
    subprocess.run([TOK_CHECK, tok_path, rq, rs], check=True, timeout=120)
    b = open(rs, "rb").read()
    at = 0

    def ids():
        nonlocal at
        n = struct.unpack_from("<I", b, at)[0]
        v = list(np.frombuffer(b, np.int64, n, at + 4))
        at += 4 + 8 * n
        return v

    def text():
        nonlocal at
        n = struct.unpack_from("<I", b, at)[0]
        v = b[at + 4:at + 4 + n]
        at += 4 + n
        return v

    enc = [(ids(), ids()) for _ in texts]
    dec = [(text(), text()) for _ in id_lists]
    assert at == len(b)
    return enc, dec


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_tokenizer_matches_reference(reflib, tmp_path, seed):
    _need(TOK_CHECK)
    path = str(tmp_path / "t.mmtok")
    pieces, _ = make_tokenizer(path, seed=seed)
    texts = random_texts(seed=seed + 10)
    rng = random.Random(seed)
    V = len(pieces)
    id_lists = [[rng.randrange(-3, V + 5) for _ in range(rng.randint(0, 30))] for _ in range(150)]
    id_lists += [[1, 2, 0], [3 + 0xE2, 3 + 0x96, 3 + 0x81, 40], [], [V, -1, 2]]
    enc, dec = ours(path, texts, id_lists, str(tmp_path))
    h = reflib.ref_tok_open(path.encode())
    assert h
    try:
        for t, (with_bos, no_bos) in zip(texts, enc):
            assert with_bos == ref_encode(reflib, h, t, True), t
            assert no_bos == ref_encode(reflib, h, t, False), t
        for ids, (skip, keep) in zip(id_lists, dec):
            assert skip == ref_decode(reflib, h, ids, True), ids
            assert keep == ref_decode(reflib, h, ids, False), ids
    finally:
        reflib.ref_tok_close(h)


def test_tokenizer_round_trip_on_valid_text(tmp_path):
    """decode(encode(t)) == t for valid UTF-8 without a leading space (the dummy prefix is
    stripped) when every merge result is a vocabulary piece, as in a real tokenizer file:
    characters outside the vocabulary come back byte for byte. (A merge into a non-piece
    falls back to the piece's bytes, U+2581 included, which decode does not turn back into
    a space -- the reference's behaviour too.)"""
    _need(TOK_CHECK)
    path = str(tmp_path / "t.mmtok")
    make_tokenizer(path, seed=5, junk_merges=0)
    texts = [t for t in random_texts(seed=6) if t and not t.startswith(b" ")]
    texts = [t for t in texts if t.decode("utf-8", "replace").encode("utf-8") == t]
    enc, _ = ours(path, texts, [], str(tmp_path))
    _, dec = ours(path, [], [e[0] for e in enc], str(tmp_path))
    for t, (s, _) in zip(texts, dec):
        assert s == t


def test_tokenizer_known_answers(tmp_path):
    """A hand-built vocabulary: merge ranks decide the segmentation, ties go left, unknown
    pieces fall back to bytes."""
    _need(TOK_CHECK)
    base = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
    extra = ["▁", "a", "b", "c", "ab", "bc", "▁a", "▁ab", "abc"]
    pieces = base + extra
    pid = {p: i for i, p in enumerate(pieces)}
    merges = ["b c", "a b", "▁ a", "▁a b", "ab c", "c c"]  # "c c" -> "cc" is not a piece
    path = str(tmp_path / "k.mmtok")
    write_mmtok(path, pieces, merges)
    enc, dec = ours(path, [b"abc", b"ab", b"cc", b"aab", b"a a"], [[pid["▁ab"], pid["c"]], [1, pid["▁a"], 2]],
                    str(tmp_path))
    # "▁abc": "b c" (rank 0) first -> ▁ a bc; then "▁ a" (rank 2) -> ▁a bc; "▁a bc" unknown
    assert enc[0][1] == [pid["▁a"], pid["bc"]]
    # "▁ab": "a b" (rank 1) before "▁ a" (rank 2) -> ▁ ab, and "▁ ab" is no merge
    assert enc[1][1] == [pid["▁"], pid["ab"]]
    # "▁cc": "c c" merges into "cc" which is not a piece -> its bytes
    assert enc[2][1] == [pid["▁"], pid["<0x63>"], pid["<0x63>"]]
    # "▁aab": "a b" (rank 1) at position 2; "▁ a" (rank 2) -> ▁a ab
    assert enc[3][1] == [pid["▁a"], pid["ab"]]
    assert enc[4][0] == [1, pid["▁a"], pid["▁a"]]
    assert dec[0][0] == b"abc"
    assert dec[1] == (b"a", b"<s> a</s>")


def test_cli_text_paths_without_model(reflib, tmp_path):
    """--decode-ids and --gen 0 --print-ids need no weights and no GPU: byte-identical to
    the reference CLI."""
    _need(CLI)
    from oracle.oracle import REF_CLI
    _need(REF_CLI)
    path = str(tmp_path / "t.mmtok")
    pieces, _ = make_tokenizer(path, seed=3)
    cases = [["--gen", "0", "--print-ids", "the quick brown fox"],
             ["--gen", "0", "--print-ids", "--no-bos", "café über naïve"],
             ["--gen", "0", "the quick"],
             ["--decode-ids", "1,300,301,302,40,2,5"],
             ["--decode-ids", ",".join(str(i) for i in range(3, 60))]]
    for extra in cases:
        args = ["--tokenizer", path] + extra
        a = subprocess.run([CLI] + args, capture_output=True, timeout=60)
        b = subprocess.run([REF_CLI] + args, capture_output=True, timeout=60)
        assert a.returncode == b.returncode == 0, (extra, a.stderr, b.stderr)
        assert a.stdout == b.stdout, extra
    # prompt from stdin
    a = subprocess.run([CLI, "--tokenizer", path, "--gen", "0", "--print-ids"], input=b"once upon a time\n\n",
                       capture_output=True, timeout=60)
    b = subprocess.run([REF_CLI, "--tokenizer", path, "--gen", "0", "--print-ids"], input=b"once upon a time\n\n",
                       capture_output=True, timeout=60)
    assert a.stdout == b.stdout and a.returncode == 0
