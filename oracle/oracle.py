"""ctypes binding of the CPU oracle (oracle/libana_oracle.so).

TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker; never by the product path.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libana_oracle.so")


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


class OrConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in
                ("vocab", "ctx", "d", "f", "layers", "heads", "rglru", "qk", "sinks", "tied")]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        vp, f32p, u64p = C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_uint64)
        sig = {
            "or_params": (C.c_uint64, [C.POINTER(OrConfig)]),
            "or_model_id": (C.c_size_t, [C.POINTER(OrConfig), C.c_char_p, C.c_size_t]),
            "or_open": (vp, [C.c_char_p, C.c_char_p, C.c_size_t]),
            "or_from_params": (vp, [C.POINTER(OrConfig), f32p]),
            "or_model_free": (None, [vp]),
            "or_model_config": (None, [vp, C.POINTER(OrConfig)]),
            "or_model_step": (C.c_uint64, [vp]),
            "or_set_threads": (None, [C.c_int]),
            "or_state_new": (vp, [vp]),
            "or_state_free": (None, [vp]),
            "or_state_clone": (vp, [vp]),
            "or_reset": (None, [vp]),
            "or_feed": (None, [vp, vp, C.c_uint32, C.c_uint32]),
            "or_logits": (None, [vp, vp, f32p]),
            "or_top": (C.c_uint32, [C.c_uint32, f32p]),
            "or_state_layer": (f32p, [vp, C.c_uint32, C.POINTER(C.c_size_t)]),
            "or_state_x": (f32p, [vp]),
            "or_tree_new": (vp, [vp]),
            "or_tree_free": (None, [vp]),
            "or_tree_step": (None, [vp, vp, C.c_uint32, C.c_uint32, f32p]),
            "or_rng_seeded": (None, [C.c_uint64, u64p]),
            "or_rng_next": (C.c_uint64, [u64p]),
            "or_u64_read": (C.c_int, [C.c_char_p, u64p]),
            "or_tree_argmax": (C.c_uint32, [C.c_uint32, f32p]),
            "or_pick": (C.c_uint32, [C.c_uint32, f32p, C.c_float, C.c_uint32, C.c_float, u64p]),
            "or_topk_threshold": (C.c_float, [C.c_uint32, f32p, C.c_uint32]),
            "or_topp_threshold": (C.c_float, [C.c_uint32, f32p, C.c_float]),
            "or_tree_sum": (C.c_float, [C.c_uint32, f32p]),
            "or_ce": (C.c_float, [C.c_uint32, f32p, C.c_uint32]),
            "or_stat": (None, [C.c_uint32, f32p, C.c_uint32, f32p, C.POINTER(C.c_uint32), f32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_float))


def to_cfg(c) -> OrConfig:
    return OrConfig(c.vocab, c.ctx, c.d, c.f, c.layers, c.heads, int(c.rglru), int(c.qk),
                    int(c.sinks), int(c.tied))


def set_threads(n: int) -> None:
    lib().or_set_threads(n)


class Model:
    """The oracle's model: from an FTC2 path or from a parameter vector."""

    def __init__(self, path: str | None = None, cfg=None, params: np.ndarray | None = None):
        L = lib()
        if path is not None:
            err = C.create_string_buffer(512)
            h = L.or_open(path.encode(), err, 512)
            if not h:
                raise ValueError(err.value.decode())
        else:
            p = np.ascontiguousarray(params, dtype=np.float32)
            oc = to_cfg(cfg)
            h = L.or_from_params(C.byref(oc), _f32p(p))
        self.h = h
        oc = OrConfig()
        L.or_model_config(h, C.byref(oc))
        self.vocab, self.ctx, self.d, self.layers = oc.vocab, oc.ctx, oc.d, oc.layers
        self.cfg = oc

    @property
    def step(self) -> int:
        return lib().or_model_step(self.h)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.or_model_free(self.h)
            self.h = None


class State:
    """One sequence on the dense engine (dd.feed / dd.logits / dd.top)."""

    def __init__(self, m: Model):
        self.m = m
        self.h = lib().or_state_new(m.h)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.or_state_free(self.h)
            self.h = None

    def reset(self) -> None:
        lib().or_reset(self.h)

    def clone(self) -> "State":
        """An independent copy of this sequence's states."""
        t = State.__new__(State)
        t.m = self.m
        t.h = lib().or_state_clone(self.h)
        return t

    def feed(self, pos: int, tok: int) -> None:
        lib().or_feed(self.m.h, self.h, pos, tok)

    def feeds(self, pos: int, toks) -> None:
        for i, t in enumerate(toks):
            self.feed(pos + i, int(t))

    def logits(self) -> np.ndarray:
        out = np.empty(self.m.vocab, dtype=np.float32)
        lib().or_logits(self.m.h, self.h, _f32p(out))
        return out

    def layer(self, l: int) -> np.ndarray:
        n = C.c_size_t()
        p = lib().or_state_layer(self.h, l, C.byref(n))
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy()

    def x(self) -> np.ndarray:
        p = lib().or_state_x(self.h)
        return np.ctypeslib.as_array(p, shape=(self.m.d,)).copy()


class Tree:
    """The meaning (bend/Model.bend decode), one token at a time."""

    def __init__(self, m: Model):
        self.m = m
        self.h = lib().or_tree_new(m.h)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.or_tree_free(self.h)
            self.h = None

    def step(self, pos: int, tok: int) -> np.ndarray:
        out = np.empty(self.m.vocab, dtype=np.float32)
        lib().or_tree_step(self.m.h, self.h, pos, tok, _f32p(out))
        return out


def top(logits: np.ndarray) -> int:
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().or_top(lg.size, _f32p(lg))


def tree_argmax(logits: np.ndarray) -> int:
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().or_tree_argmax(lg.size, _f32p(lg))


def tree_sum(x: np.ndarray) -> float:
    a = np.ascontiguousarray(x, dtype=np.float32)
    return lib().or_tree_sum(a.size, _f32p(a))


def stat(logits: np.ndarray, x: int):
    """dc.prob.of / al.stat: (p, a, pa) in the reference's tree order."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    p, a, pa = C.c_float(), C.c_uint32(), C.c_float()
    lib().or_stat(lg.size, _f32p(lg), int(x), C.byref(p), C.byref(a), C.byref(pa))
    return np.float32(p.value), int(a.value), np.float32(pa.value)


def ce(logits: np.ndarray, y: int) -> float:
    """G.lse(logits) - logits[y] in the reference's tree order."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().or_ce(lg.size, _f32p(lg), int(y))


def rng_seeded(seed: int) -> np.ndarray:
    r = np.zeros(4, dtype=np.uint64)
    lib().or_rng_seeded(seed, r.ctypes.data_as(C.POINTER(C.c_uint64)))
    return r


def rng_next(r: np.ndarray) -> int:
    return lib().or_rng_next(r.ctypes.data_as(C.POINTER(C.c_uint64)))


def u64_read(s: str):
    out = C.c_uint64()
    ok = lib().or_u64_read(s.encode(), C.byref(out))
    return out.value if ok else None


def pick(logits: np.ndarray, temp: float, topk: int, topp: float, rng: np.ndarray) -> int:
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().or_pick(lg.size, _f32p(lg), temp, topk, topp, rng.ctypes.data_as(C.POINTER(C.c_uint64)))


def topk_threshold(logits: np.ndarray, k: int) -> float:
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().or_topk_threshold(lg.size, _f32p(lg), k)


def topp_threshold(w: np.ndarray, p: float) -> float:
    a = np.ascontiguousarray(w, dtype=np.float32)
    return lib().or_topp_threshold(a.size, _f32p(a), p)


def params(cfg) -> int:
    oc = to_cfg(cfg)
    return lib().or_params(C.byref(oc))


def model_id(cfg) -> str:
    oc = to_cfg(cfg)
    buf = C.create_string_buffer(1024)
    n = lib().or_model_id(C.byref(oc), buf, 1024)
    return buf.value[:n].decode()
