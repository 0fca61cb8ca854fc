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


def test_eight_effects_declared():
    names = [d[0] for d in DEFS]
    assert names == ["ana.open", "ana.reset", "ana.feed", "ana.feeds", "ana.logits", "ana.top", "ana.pick",
                     "ana.score"], names


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
