"""The host-side BPE tokenizer (bend/Tokenizer.bend, bend/Sha256.bend) in
libana, on the CPU.

It is pinned by:
- SHA-256 against the FIPS 180-4 vectors that tests/sha.bend prints, against
  hashlib at the padding edges, and against weights/SHA256SUMS for the two
  artifacts (tests/golden/bpe holds those files, which tests/tok.bend reads);
- the identity string against a restatement over hashlib;
- pretokenization against a restatement of the Bend definitions, itself
  pinned by hand-derived splits under both rules;
- encoding against a brute-force restatement of encode.word.ref (the
  reference's slow algorithm: the lowest merge id among adjacent pairs
  replaces every occurrence, left to right), on both artifacts and on a
  synthetic one with a duplicated pair;
- decode(encode(x)) == x on random byte strings.
"""
import hashlib
import os

import numpy as np
import pytest

import ana_amd

HERE = os.path.dirname(os.path.abspath(__file__))
BPE = os.path.join(HERE, "golden", "bpe")
ARTS = ["enwiki-fineweb-32k.bpe", "code32k.bpe"]


def _sums():
    out = {}
    for ln in open(os.path.join(BPE, "SHA256SUMS")):
        h, name = ln.split()
        out[name] = h
    return out


def test_sha256_vectors():
    # FIPS 180-4's examples (tests/sha.bend prints these three digests)
    assert ana_amd.sha256_hex(b"") == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"
    assert ana_amd.sha256_hex(b"abc") == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert ana_amd.sha256_hex(b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq") == \
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"
    rng = np.random.default_rng(5)
    for n in (1, 55, 56, 57, 63, 64, 65, 119, 120, 128, 1000):
        b = rng.integers(0, 256, size=n).astype(np.uint8).tobytes()
        assert ana_amd.sha256_hex(b) == hashlib.sha256(b).hexdigest(), n


def test_artifacts_match_their_sums():
    sums = _sums()
    for a in ARTS:
        assert ana_amd.sha256_hex(open(os.path.join(BPE, a), "rb").read()) == sums[a]


def _rows(path):
    lines = open(path, "rb").read().split(b"\n")
    head = lines[0].split()
    vocab, v2 = int(head[1]), len(head) > 2 and head[2] == b"v2"
    merges = [tuple(int(x) for x in ln.split()) for ln in lines[1:] if ln.strip()]
    return vocab, v2, merges


def test_identity_restated():
    # Bpe.identity (bend/Tokenizer.bend:307-336), restated over hashlib
    for a in ARTS:
        vocab, v2, merges = _rows(os.path.join(BPE, a))
        canon = f"fastbpe-word-v1\nvocab {vocab}\n" + "".join(f"{x} {y} {z}\n" for x, y, z in merges)
        rule = "ascii-space-run+lf-prefix-v2" if v2 else "ascii-space-prefix+lf-boundary"
        want = (f"fastbpe-word-v1:bos=0:eos=1:bytes=2..257:pretoken={rule}:vocab={vocab}:sha256="
                + hashlib.sha256(canon.encode()).hexdigest())
        t = ana_amd.Tokenizer(os.path.join(BPE, a))
        assert t.vocab == vocab
        assert t.identity() == want


# ---- restatements (test side) of pretokenize and encode.word.ref ----

def _ordinary(c):
    return c != 32 and c != 10


def _span_ord(xs, i):
    j = i
    while j < len(xs) and _ordinary(xs[j]):
        j += 1
    return j


def pretok(xs, v2):
    """bend/Tokenizer.bend:338-472 as lists of byte lists."""
    xs = list(xs)
    out, i = [], 0
    while i < len(xs):
        h = xs[i]
        if not v2:
            if h == 10:
                out.append([10]); i += 1
            elif h == 32:
                j = _span_ord(xs, i + 1); out.append(xs[i:j]); i = j
            else:
                j = _span_ord(xs, i); out.append(xs[i:j]); i = j
            continue
        if h != 10 and h != 32:
            j = _span_ord(xs, i); out.append(xs[i:j]); i = j
            continue
        lead = [10] if h == 10 else []
        k = i + 1 if h == 10 else i
        sp = []
        while k < len(xs) and xs[k] == 32:
            sp.append(32); k += 1
        if k < len(xs) and _ordinary(xs[k]):
            first = lead + sp[:-1]
            if first:
                out.append(first)
            j = _span_ord(xs, k)
            out.append(sp[-1:] + xs[k:j]); i = j
        else:
            out.append(lead + sp); i = k
    return out


def _enc_ref(word, rank):
    """encode.word.ref: repeatedly the lowest merge id among adjacent pairs,
    every occurrence replaced left to right without overlap."""
    xs = [b + 2 for b in word]
    while True:
        m = min((rank.get((xs[i], xs[i + 1]), 1 << 32) for i in range(len(xs) - 1)), default=1 << 32)
        if m == 1 << 32:
            return xs
        ys, i = [], 0
        a, b = None, None
        for (x, y), z in rank.items():
            if z == m:
                a, b = x, y
        while i < len(xs):
            if i + 1 < len(xs) and xs[i] == a and xs[i + 1] == b:
                ys.append(m); i += 2
            else:
                ys.append(xs[i]); i += 1
        xs = ys


def _rank_of(merges):
    rank = {}
    for x, y, z in merges:
        rank[(x, y)] = z   # the latest id of a pair wins (rank.first over a latest-first list)
    return rank


@pytest.mark.parametrize("v2", [False, True], ids=["v1", "v2"])
def test_pretokenize_hand_cases(v2):
    def words(s):
        return [bytes(w).decode() for w in pretok(s.encode(), v2)]
    assert words("  two  spaces\nand a newline") == [" ", " two", " ", " spaces", "\n", "and", " a", " newline"]
    if v2:
        assert words("a   b") == ["a", "  ", " b"]
        assert words("a  ") == ["a", "  "]
        assert words("\n  x") == ["\n ", " x"]
        assert words("\n\n") == ["\n", "\n"]
        assert words("\nx") == ["\n", "x"]
    else:
        assert words("a   b") == ["a", " ", " ", " b"]
        assert words("a  ") == ["a", " ", " "]
        assert words("\n  x") == ["\n", " ", " x"]
        assert words("\n\n") == ["\n", "\n"]


def _random_text(rng, n):
    alpha = list(b"aeiou tnsrl\n") + [32, 32, 32]
    return bytes(int(alpha[i]) for i in rng.integers(0, len(alpha), size=n))


@pytest.mark.parametrize("art", ARTS)
def test_encode_matches_reference_algorithm(art):
    path = os.path.join(BPE, art)
    _, v2, merges = _rows(path)
    rank = _rank_of(merges)
    t = ana_amd.Tokenizer(path)
    rng = np.random.default_rng(11)
    cases = [b"The history of", b"Albert Einstein was", b"In mathematics, a group is",
             b"The city of Paris", b"Water is", b"  two  spaces\nand a newline"]
    cases += [_random_text(rng, int(rng.integers(1, 80))) for _ in range(60)]
    for s in cases:
        want = [i for w in pretok(s, v2) for i in _enc_ref(w, rank)]
        got = t.encode(s)
        assert list(got) == want, s
        assert t.decode(got) == s


def test_synthetic_artifact(tmp_path):
    # a duplicated pair (the later id wins) and overlapping occurrences
    # ("aaaa": (a, a) merges left to right without overlap)
    a, sp = 97 + 2, 32 + 2
    rows = [(a, a, 258), (258, 258, 259), (sp, a, 260), (a, a, 261)]
    p = tmp_path / "s.bpe"
    p.write_text("BPE 262 v2\n" + "".join(f"{x} {y} {z}\n" for x, y, z in rows))
    t = ana_amd.Tokenizer(str(p))
    rank = _rank_of(rows)
    for s in (b"aaaa", b"aaa", b"a aaaaa", b"  aa", b"aaaaaaa"):
        want = [i for w in pretok(s, True) for i in _enc_ref(w, rank)]
        assert list(t.encode(s)) == want, s
        assert t.decode(t.encode(s)) == s


def test_round_trip_random_bytes():
    rng = np.random.default_rng(12)
    toks = [ana_amd.Tokenizer(os.path.join(BPE, a)) for a in ARTS] + [ana_amd.Tokenizer(None)]
    for _ in range(40):
        s = rng.integers(0, 256, size=int(rng.integers(0, 300))).astype(np.uint8).tobytes()
        for t in toks:
            assert t.decode(t.encode(s)) == s
    b = ana_amd.Tokenizer(None)
    assert b.vocab == 258
    assert list(b.encode(b"hi\n")) == [104 + 2, 105 + 2, 10 + 2]
    assert b.decode([0, 1, 106, 107]) == b"hi"   # BOS and EOS give no bytes


def test_parse_rejections(tmp_path):
    bad = {"gap": "BPE 260\n1 2 258\n3 4 260\n", "count": "BPE 261\n1 2 258\n3 4 259\n",
           "header": "XPE 259\n1 2 258\n", "blank": "BPE 259\n1 2 258\n\n"}
    for name, text in bad.items():
        p = tmp_path / f"{name}.bpe"
        p.write_text(text)
        with pytest.raises(ana_amd.AnaError):
            ana_amd.Tokenizer(str(p))
    ok = tmp_path / "ok.bpe"
    ok.write_text("BPE 259\r\n  1 2 258 trailing words\n")
    assert ana_amd.Tokenizer(str(ok)).vocab == 259


def test_find_tokenizer(tmp_path):
    paths = [os.path.join(BPE, a) for a in ARTS]
    want = ana_amd.Tokenizer(paths[1]).identity()
    assert ana_amd.find_tokenizer(want, candidates=paths).identity() == want
    assert ana_amd.find_tokenizer(ana_amd.BYTE_IDENTITY).vocab == 258
    with pytest.raises(ana_amd.AnaError, match="TOKENIZER_FILE identity does not match"):
        ana_amd.find_tokenizer(want, pinned=paths[0])
    with pytest.raises(ana_amd.AnaError, match="no candidate tokenizer matches"):
        ana_amd.find_tokenizer(want + "x", candidates=paths)


def test_manifest_round_trip_and_discovery(tmp_path):
    """Every manifest field through ckpt.write and ana_manifest_read (the
    doubles as F32), and the checkpoint's tokenizer found by identity."""
    from ana_amd import ckpt, config as cf
    tok = ana_amd.Tokenizer(os.path.join(BPE, "code32k.bpe"))
    p = str(tmp_path / "m.ftc2")
    c = cf.SMALL4_V3
    ckpt.write(p, c, ckpt.init_params(c, "hash"), tokenizer_id=tok.identity(), dataset_id="enwik8-test",
               adamw=(6.0e-4, 0.9, 0.98, 1.0e-9, 0.05, 200, 12000), muon=0.02, clip=0.5, numerics=1)
    m = ana_amd.read_manifest(p)
    f32 = np.float32
    assert (m["version"], m["count"], m["layout"], m["layout_version"]) == \
        (4, c.params, "hybrid-gla-decoder-flat-parameters", 3)
    assert m["cfg"] == {"vocab": 258, "ctx": 64, "d": 64, "f": 192, "layers": 4, "heads": 4,
                        "rglru": 1, "qk": 1, "sinks": 1, "tied": 1}
    assert [f32(m[k]) for k in ("lr", "beta1", "beta2", "eps", "weight_decay")] == \
        [f32(6.0e-4), f32(0.9), f32(0.98), f32(1.0e-9), f32(0.05)]
    assert (m["warmup"], m["total_steps"], m["has_muon"], f32(m["muon"])) == (200, 12000, True, f32(0.02))
    assert (m["model_id"], m["dataset_id"], f32(m["clip"]), m["numerics"]) == \
        (c.model_id, "enwik8-test", f32(0.5), 1)
    assert ana_amd.find_tokenizer(m["tokenizer_id"],
                                  candidates=[os.path.join(BPE, a) for a in ARTS]).identity() == tok.identity()


def test_manifest_big_integer_double(tmp_path):
    """Load.double with a big Integer mantissa (a Double's decodeFloat, as
    the Haskell master writes it): sign byte, byte count, little-endian
    bytes, folded in F32 by le.f32, times F32.pow(2, e)."""
    import math
    import struct
    from ana_amd import ckpt, config as cf
    c = cf.SMALL4_V3
    base = ckpt.manifest_bytes(c)
    lr = ckpt._double(3.0e-4)
    i = base.index(lr)
    fr, ex = math.frexp(3.0e-4)
    mant, e = int(fr * (1 << 53)), ex - 53
    bs = mant.to_bytes((mant.bit_length() + 7) // 8, "little")
    big = b"\x01" + b"\x01" + struct.pack(">Q", len(bs)) + bs + struct.pack(">q", e)
    p = tmp_path / "b.ftc2"
    p.write_bytes(base[:i] + big + base[i + len(lr):])
    want = np.float32(0.0)
    for b in reversed(bs):
        want = np.float32(np.float32(b) + np.float32(np.float32(256.0) * want))
    want = np.float32(want * np.float32(2.0 ** e))
    got = ana_amd.read_manifest(str(p))["lr"]
    assert np.float32(got) == want
    assert abs(got - 3.0e-4) <= 1e-6 * 3.0e-4
    with pytest.raises(ana_amd.AnaError, match="magic"):
        q = tmp_path / "x.ftc2"
        q.write_bytes(b"XXXX" + base[4:])
        ana_amd.read_manifest(str(q))
