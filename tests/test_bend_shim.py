"""The Bend binding (bend/AnaIo.bend, bend/effs/ana.c) against itself and
the C ABI. Bend is not installed here, so neither file compiles in this
image; these checks hold what can be held by reading: every declared
effect has its handler registered under the same name, every handler
reads the argument positions its declaration has, and every library
symbol the handlers resolve is one include/ana.h declares and libana
exports (the reference's effect interface: BulkIo.bend:16-93 declares,
bulk.c:2586-2822 registers)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BEND = open(os.path.join(ROOT, "bend", "AnaIo.bend")).read()
C = open(os.path.join(ROOT, "bend", "effs", "ana.c")).read()
HDR = open(os.path.join(ROOT, "include", "ana.h")).read()

DEFS = re.findall(r"^def (ana\.[a-z_]+)\((.*?)\) -> IO\((.*?)\):\n  import \"\./effs/ana\.c\"", BEND, re.M)


def test_nine_effects_declared():
    names = [d[0] for d in DEFS]
    assert names == ["ana.open", "ana.step", "ana.reset", "ana.feed", "ana.feeds", "ana.logits", "ana.top",
                     "ana.pick", "ana.score"], names


@pytest.mark.parametrize("name,args,ret", DEFS)
def test_handler_registered_and_reads_its_arguments(name, args, ret):
    fn = name.replace(".", "_") + "_run"
    block = re.search(r"#ifdef CID\(%s\)\n(.*?)#endif" % re.escape(name), C, re.S)
    assert block, f"no #ifdef CID({name}) block"
    body = block.group(1)
    assert f"Term {fn}(Env e, Term* f, IoWork* w)" in body
    assert f"io_eff(CID({name}), {fn});" in body
    # the highest argument index the handler reads is its last parameter
    n = len([a for a in args.split(",") if a.strip()])
    used = {int(i) for i in re.findall(r"\bf\[(\d+)\]", body)}
    assert used == set(range(n)), (name, sorted(used), n)
    # a pair result is built with io_tup, a single one is returned as is
    assert ("io_tup(" in body) == ("&" in ret), (name, ret)


def test_strings_read_as_bulk_c_reads_them():
    # io_cbuf's four arguments (bulk.c:2502): env, term, length out, SCon
    calls = re.findall(r"io_cbuf\(([^;]*)\);", C)
    assert calls and all(len([x for x in c.split(",")]) == 4 and c.endswith("CID(SCon)") for c in calls), calls


def test_resolved_symbols_are_the_abi():
    syms = re.findall(r'an_sym\(lib, "([a-z_0-9]+)"\)', C)
    assert len(syms) == 10, syms
    for s in syms:
        assert re.search(r"\b%s\(" % s, HDR), f"{s} not declared in include/ana.h"
    so = os.path.join(ROOT, "ana_amd", "libana.so")
    if not os.path.exists(so):
        pytest.skip("libana.so not built")
    lib = ctypes.CDLL(so)
    for s in syms:
        assert hasattr(lib, s), s


# ---- the engine arm: bend/Decode.bend.ana.patch
PATCH_PATH = os.path.join(ROOT, "bend", "Decode.bend.ana.patch")
PATCH = open(PATCH_PATH).read()
REF_DECODE = "/root/reference/bend/Decode.bend"

# each seam function of Decode.bend (En's cases, bend/Decode.bend:304-470)
# and what its EAna arm must reach: the library effect, or the engine
# helper that reaches it
SEAM = {
    "dc.en.step": ["AI.ana.feed(", "dc.en.ana.io("],
    "dc.en.feed": ["AI.ana.feed("],
    "dc.en.feeds": ["dc.en.ana.ids("],
    "dc.en.prefill": ["dc.en.ana.prefill("],
    "dc.en.step.pick": ["AI.ana.feed(", "dc.en.ana.pick("],
    "dc.en.prefill.pick": ["dc.en.ana.prefill.pick("],
    "dc.en.reset": ["AI.ana.reset("],
    "dc.en.name": ['"ana"'],
}
# the engine's helpers and the effects they reach
HELPERS = {
    "dc.en.ana.io": ["AI.ana.logits("],
    "dc.en.ana.ids": ["AI.ana.feeds(", "DIo.put.u32("],
    "dc.en.ana.prefill": ["dc.en.ana.ids(", "dc.en.ana.io("],
    "dc.en.ana.pick": ["AI.ana.top(", "dc.en.ana.io("],
    "dc.en.ana.prefill.pick": ["dc.en.ana.ids(", "dc.en.ana.pick("],
    "dc.loaded.ana": ["AI.ana.open(", "AI.ana.step(", "EAna{"],
    "dc.load.eng.of": ["dc.loaded.ana(", "dc.load.fmt("],
}


def _defs(text):
    """{name: body} of every top-level def in text"""
    out, cur, body = {}, None, []
    for line in text.split("\n"):
        m = re.match(r"def ([a-z_.]+)\(", line)
        if m:
            if cur:
                out[cur] = "\n".join(body)
            cur, body = m.group(1), [line]
        elif cur is not None:
            if line and not line.startswith(" "):
                out[cur] = "\n".join(body)
                cur, body = None, []
            else:
                body.append(line)
    if cur:
        out[cur] = "\n".join(body)
    return out


def test_patch_adds_only_its_own_lines():
    """A zero-context diff: every hunk inserts, except the one line of
    dc.load that now asks dc.load.eng."""
    minus = [l for l in PATCH.split("\n") if l.startswith("-") and not l.startswith("---")]
    assert minus == ['-    dc.load.fmt(String.ends_with(path, ".btc"), String.eq(eng, "tree"), path, pinned)'], minus
    assert "+    dc.load.eng(eng, path, pinned)" in PATCH
    assert "+  EAna{h: U32, q: U32, dv: Nat, v: U32, x: Array<F32>}" in PATCH
    assert "+import ./AnaIo.bend as AI" in PATCH


def test_patch_effects_are_declared():
    used = set(re.findall(r"AI\.(ana\.[a-z_]+)\(", PATCH))
    declared = {d[0] for d in DEFS}
    assert used and used <= declared, used - declared


def _patched():
    import shutil
    import subprocess
    import tempfile
    if not os.path.exists(REF_DECODE):
        pytest.skip("the reference tree is not here")
    d = tempfile.mkdtemp()
    os.makedirs(os.path.join(d, "bend"))
    shutil.copy(REF_DECODE, os.path.join(d, "bend", "Decode.bend"))
    r = subprocess.run(["git", "apply", "--unidiff-zero", PATCH_PATH], cwd=d, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return open(os.path.join(d, "bend", "Decode.bend")).read()


def test_patch_applies_and_every_seam_case_has_its_arm():
    text = _patched()
    defs = _defs(text)
    for fn, calls in SEAM.items():
        body = defs[fn]
        assert "case EAna{" in body, fn
        arm = body[body.index("case EAna{"):]
        for c in calls:
            assert c in arm, (fn, c)
    for fn, calls in HELPERS.items():
        assert fn in defs, fn
        for c in calls:
            assert c in defs[fn], (fn, c)
    # the engines' other arms are untouched, and dc.load chooses by ANA_DECODER
    for fn in SEAM:
        assert "case EDense{" in defs[fn] and "case ETree{" in defs[fn], fn
    assert 'String.eq(eng, "hip")' in defs["dc.load.eng"]
    assert "dc.load.eng(eng, path, pinned)" in defs["dc.load"]
