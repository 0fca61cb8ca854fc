"""ana_generate_noalloc, the token loop that allocates nothing (its
scratch is a fixed device array), against ana_generate through the C ABI:
the same picks and RNG words bit for bit in exact mode, greedy and sampled,
on two calls in a row on the same contexts, the second smaller; and a call
too large for the array fails with ANA_EINVAL."""
import ctypes as C
import json
import os

import numpy as np
import pytest

import ana_amd
from ana_amd import ckpt
from ana_amd import config as cf

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
VEC = json.load(open(os.path.join(HERE, "golden", "reference_vectors.json")))


def _u32p(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def _call(fn, dec, seqs, pos, tok, steps, st, rng):
    s = np.ascontiguousarray(seqs, dtype=np.uint32)
    p = np.ascontiguousarray(pos, dtype=np.uint32)
    t = np.ascontiguousarray(tok, dtype=np.uint32)
    out = np.zeros((s.size, steps), dtype=np.uint32)
    sp = C.byref(st._c()) if st is not None else None
    rp = rng.ctypes.data_as(C.POINTER(C.c_uint64)) if rng is not None else None
    r = fn(dec.h, s.size, _u32p(s), _u32p(p), _u32p(t), steps, sp, rp, _u32p(out))
    return r, out


@pytest.mark.parametrize("sampled", [False, True], ids=["greedy", "sampled"])
@pytest.mark.parametrize("mode", [ana_amd.EXACT_FP32, ana_amd.FAST_FP32], ids=["exact", "fast_fp32"])
def test_generate_noalloc_equals_generate(tmp_path, mode, sampled):
    print(f"case generate_noalloc mode {mode} sampled {sampled}", flush=True)
    c = cf.SMALL4_V3
    path = str(tmp_path / "na.ftc2")
    ckpt.write(path, c, ckpt.init_params(c, "hash", 1, trained=True))
    L = ana_amd.lib()
    st = ana_amd.Settings(float(np.float32(0.8)), 40, float(np.float32(0.9))) if sampled else None
    n0 = 6
    prompts = [VEC["window"][5 * i: 5 * i + 3 + i] for i in range(n0)]
    with ana_amd.Decoder(path, max_seqs=n0, prefill_chunk=8, numerics=mode) as a, \
            ana_amd.Decoder(path, max_seqs=n0, prefill_chunk=8, numerics=mode) as b:
        for d in (a, b):
            d.feeds_n(list(range(n0)), [0] * n0, [pr[:-1] for pr in prompts])
        pos = np.array([len(pr) - 1 for pr in prompts], dtype=np.uint32)
        tok = np.array([pr[-1] for pr in prompts], dtype=np.uint32)
        # two calls in a row, the second with fewer rows and steps (from
        # where each row stopped)
        for seqs, steps in ((list(range(n0)), 40), ([4, 1, 3], 9)):
            idx = np.array(seqs)
            rng = (np.ascontiguousarray(np.stack([ana_amd.rng_seeded(70 + q) for q in seqs]).astype(np.uint64))
                   if sampled else None)
            rng2 = rng.copy() if sampled else None
            ra, oa = _call(L.ana_generate, a, seqs, pos[idx], tok[idx], steps, st, rng)
            rb, ob = _call(L.ana_generate_noalloc, b, seqs, pos[idx], tok[idx], steps, st, rng2)
            assert ra == 0 and rb == 0, (ra, rb, L.ana_error(b.h))
            assert np.array_equal(oa, ob), (seqs, steps)
            if sampled:
                assert np.array_equal(rng, rng2)
            pos[idx] += steps
            tok[idx] = oa[:, -1]
        # the residual rows both calls leave behind agree too (ana_logits)
        assert np.array_equal(a.logits([0, 1, 2]).view(np.uint32), b.logits([0, 1, 2]).view(np.uint32)) \
            or mode != ana_amd.EXACT_FP32
        # beyond the array: 2^18 words hold at most (2^18 - 64) / 2 picks
        r, _ = _call(L.ana_generate_noalloc, b, [0], [int(pos[0])], [int(tok[0])], 140000, None, None)
        assert r == ana_amd.ANA_EINVAL and "scratch words" in L.ana_error(b.h).decode()
