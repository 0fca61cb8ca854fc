"""The C ABI without a GPU: libana.so loads, exports every function
include/ana.h declares, and rejects bad checkpoints with the reference's
messages before touching a device (bend/Checkpoint.bend:162-170,
bend/Dense/Decode.bend:664-699)."""
import ctypes as C
import os
import re
import struct

import numpy as np
import pytest

import ana_amd
from ana_amd import ckpt
from ana_amd import config as cf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "ana.h")).read()
    return sorted(set(re.findall(r"\b(ana_[a-z_0-9]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    L = ana_amd.lib()
    names = header_functions()
    assert "ana_open" in names and "ana_generate" in names
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(ana_amd.SIGNATURES)


def _open_err(path):
    L = ana_amd.lib()
    h = C.c_void_p()
    o = ana_amd._Opts(0, 0, 1, 64)
    r = L.ana_open(path.encode(), C.byref(o), C.byref(h))
    return r, L.ana_error(None).decode()


@pytest.fixture()
def good(tmp_path):
    c = cf.SMALL4_V3
    path = str(tmp_path / "g.ftc2")
    ckpt.write(path, c, ckpt.init_params(c, "normal", 1))
    return path, open(path, "rb").read()


def test_rejects_bad_checkpoints(tmp_path, good):
    path, raw = good
    bad = tmp_path / "b.ftc2"

    bad.write_bytes(b"XTC2" + raw[4:])
    assert _open_err(str(bad)) == (ana_amd.ANA_ECKPT, "not a compact checkpoint (magic is not FTC2)")

    bad.write_bytes(raw[:4] + struct.pack(">I", 3) + raw[8:])
    r, msg = _open_err(str(bad))
    assert r == ana_amd.ANA_ECKPT and "manifest version" in msg

    bad.write_bytes(raw[: len(raw) - 9])
    assert _open_err(str(bad)) == (ana_amd.ANA_ECKPT, "checkpoint: short read")

    # a manifest count that is not Config.params
    c = cf.SMALL4_V3
    m = ckpt.manifest_bytes(c)
    off = 4 + 4 + 6 * 8 + 4
    assert struct.unpack(">Q", m[off:off + 8])[0] == c.params
    bad.write_bytes(raw[:off] + struct.pack(">Q", c.params + 1) + raw[off + 8:])
    r, msg = _open_err(str(bad))
    assert r == ana_amd.ANA_ECKPT and msg == "checkpoint: manifest parameter count does not match config"

    # an untied head is refused by the dense decoder
    u = cf.Config(c.vocab, c.ctx, c.d, c.f, c.layers, c.heads, True, True, True, False)
    ckpt.write(str(bad), u, ckpt.init_params(u, "normal", 1))
    assert _open_err(str(bad)) == (ana_amd.ANA_ECKPT, "checkpoint: the dense decoder needs a tied head")

    # the parameter vector's own count
    h = len(ckpt.manifest_bytes(c))
    bad.write_bytes(raw[:h] + struct.pack(">Q", 7) + raw[h + 8:])
    assert _open_err(str(bad)) == (
        ana_amd.ANA_ECKPT, "checkpoint: checkpoint parameter vector length is not the parameter count")


def test_settings_semantics():
    s = ana_amd.settings("0.8", "", "0.95")
    assert s.top_k == 0xFFFFFFFF and abs(s.temperature - 0.8) < 1e-7 and not s.greedy
    assert ana_amd.settings("abc", "x", "y") == ana_amd.settings()
    assert ana_amd.settings("0", "40", "0.9").greedy
    assert ana_amd.u64_read("18446744073709551615") == 2 ** 64 - 1
    assert ana_amd.u64_read("-1") is None


def test_rng_seeded_matches_oracle(oracle):
    for seed in (0, 1, 2 ** 40 + 3):
        assert np.array_equal(ana_amd.rng_seeded(seed), oracle.rng_seeded(seed))


def test_truncate_at_eos():
    assert list(ana_amd.truncate_at_eos(np.array([5, 7, 1, 9]))) == [5, 7, 1]
    assert list(ana_amd.truncate_at_eos(np.array([5, 7]))) == [5, 7]
