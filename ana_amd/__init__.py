"""ana_amd: hhefesto/ana's decoder token loop on MI355X.

The product is libana.so (ana_amd/csrc, C ABI in include/ana.h). This module
is a thin ctypes mirror of the engine seam the reference's host code drives
(bend/Decode.bend's dc.* over bend/Dense/Decode.bend's dd.*): load, reset,
feed, feeds, logits, top, pick, and the token loop. It never computes
anything itself and raises if libana.so is missing.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from .config import Config

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libana.so")

ANA_OK, ANA_EINVAL, ANA_ECKPT, ANA_EDEVICE, ANA_ENOMEM, ANA_EUNSUP, ANA_ETOK, ANA_ETIME = range(8)
EXACT_FP32 = 0
FAST_FP32 = 1
BF16 = 2
EOS = 1  # bend/Tokenizer.bend: BOS 0, EOS 1


class AnaError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class _Cfg(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in
                ("vocab", "ctx", "d", "f", "layers", "heads", "rglru", "qk", "sinks", "tied")]


_MSTR = 1024


class _Manifest(C.Structure):
    _fields_ = [("version", C.c_uint32), ("cfg", _Cfg), ("count", C.c_uint32),
                ("layout", C.c_char * _MSTR), ("layout_version", C.c_uint32),
                ("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
                ("weight_decay", C.c_float), ("warmup", C.c_uint32), ("total_steps", C.c_uint32),
                ("has_muon", C.c_uint32), ("muon", C.c_float),
                ("model_id", C.c_char * _MSTR), ("tokenizer_id", C.c_char * _MSTR),
                ("dataset_id", C.c_char * _MSTR), ("clip", C.c_float), ("numerics", C.c_uint32)]


class _Opts(C.Structure):
    _fields_ = [("device", C.c_int), ("numerics", C.c_int), ("max_seqs", C.c_uint32),
                ("prefill_chunk", C.c_uint32)]


class _Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float)]


# every symbol include/ana.h declares, with its signature
_u32p = C.POINTER(C.c_uint32)
_u64p = C.POINTER(C.c_uint64)
_f32p = C.POINTER(C.c_float)
SIGNATURES = {
    "ana_open": (C.c_int, [C.c_char_p, C.POINTER(_Opts), C.POINTER(C.c_void_p)]),
    "ana_config_of": (C.c_int, [C.c_void_p, C.POINTER(_Cfg), _u64p]),
    "ana_reset": (C.c_int, [C.c_void_p, C.c_uint32]),
    "ana_feed": (C.c_int, [C.c_void_p, C.c_uint32, _u32p, _u32p, _u32p]),
    "ana_feeds": (C.c_int, [C.c_void_p, C.c_uint32, C.c_uint32, _u32p, C.c_uint32]),
    "ana_feeds_n": (C.c_int, [C.c_void_p, C.c_uint32, _u32p, _u32p, _u32p, _u32p]),
    "ana_score_n": (C.c_int, [C.c_void_p, C.c_uint32, _u32p, _u32p, _u32p, _u32p, _f32p]),
    "ana_logits": (C.c_int, [C.c_void_p, C.c_uint32, _u32p, _f32p]),
    "ana_top": (C.c_int, [C.c_void_p, C.c_uint32, _u32p, _u32p]),
    "ana_stats": (C.c_int, [C.c_void_p, C.c_uint32, _u32p, _u32p, _f32p, _u32p, _f32p]),
    "ana_pick": (C.c_int, [C.c_void_p, C.c_uint32, _u32p, C.POINTER(_Sampling), _u64p, _u32p]),
    "ana_rng_seeded": (None, [C.c_uint64, _u64p]),
    "ana_generate": (C.c_int, [C.c_void_p, C.c_uint32, _u32p, _u32p, _u32p, C.c_uint32,
                               C.POINTER(_Sampling), _u64p, _u32p]),
    "ana_generate_noalloc": (C.c_int, [C.c_void_p, C.c_uint32, _u32p, _u32p, _u32p, C.c_uint32,
                                       C.POINTER(_Sampling), _u64p, _u32p]),
    "ana_state": (C.c_int, [C.c_void_p, C.c_uint32, C.c_uint32, _f32p, C.c_size_t]),
    "ana_prof": (C.c_int, [C.c_void_p, C.c_int]),
    "ana_prof_read": (C.c_int, [C.c_void_p, C.c_uint32, _u64p, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "ana_trace": (C.c_int, [C.c_void_p, C.c_uint32]),
    "ana_trace_read": (C.c_int, [C.c_void_p, _u32p, C.c_size_t, _u32p]),
    "ana_probe_reread": (C.c_int, [C.c_int, C.c_uint64, C.c_uint32, C.POINTER(C.c_double)]),
    "ana_bpe_open": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "ana_bpe_bytes": (C.c_int, [C.POINTER(C.c_void_p)]),
    "ana_bpe_close": (None, [C.c_void_p]),
    "ana_bpe_vocab": (C.c_uint32, [C.c_void_p]),
    "ana_bpe_identity": (C.c_int, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "ana_bpe_encode": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint8), C.c_size_t, _u32p, C.c_size_t,
                                 C.POINTER(C.c_size_t)]),
    "ana_bpe_decode": (C.c_int, [C.c_void_p, _u32p, C.c_size_t, C.POINTER(C.c_uint8), C.c_size_t,
                                 C.POINTER(C.c_size_t)]),
    "ana_sha256_hex": (C.c_int, [C.POINTER(C.c_uint8), C.c_size_t, C.c_char_p]),
    "ana_manifest_read": (C.c_int, [C.c_char_p, C.c_void_p]),
    "ana_error": (C.c_char_p, [C.c_void_p]),
    "ana_close": (None, [C.c_void_p]),
}

_lib = None


def lib() -> C.CDLL:
    """libana.so, loaded once; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (or python ana_amd/build.py)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32).reshape(-1))


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(C.POINTER(t))


@dataclass
class Settings:
    """bend/Decode.bend:147-148: temperature, top-k (off = 2^32-1), top-p."""

    temperature: float = float(np.float32(0.8))
    top_k: int = 0xFFFFFFFF
    top_p: float = float(np.float32(0.95))

    @property
    def greedy(self) -> bool:
        return self.temperature <= 0.0

    def _c(self) -> _Sampling:
        return _Sampling(self.temperature, self.top_k, self.top_p)


def _f32_or(s: str, d: float) -> float:
    try:
        return float(np.float32(float(s)))
    except ValueError:
        return float(np.float32(d))


def settings(temp: str = "0.8", topk: str = "", topp: str = "0.95") -> Settings:
    """dc.settings (bend/Decode.bend:546-548): non-numeric values fall back
    to the defaults TEMPERATURE 0.8, TOP_K off, TOP_P 0.95."""
    k = int(topk) if topk.isdigit() and int(topk) < 2 ** 32 else 0xFFFFFFFF
    return Settings(_f32_or(temp, 0.8), k, _f32_or(topp, 0.95))


def u64_read(s: str):
    """U64.read (bend/Num.bend:147-170): digits only, wrapping; None otherwise."""
    if not s or not s.isdigit() or not s.isascii():
        return None
    v = 0
    for ch in s:
        v = (v * 10 + ord(ch) - 48) & 0xFFFFFFFFFFFFFFFF
    return v


def rng_seeded(seed: int) -> np.ndarray:
    """Rng.seeded (bend/Sample.bend:68-93): 4 xoshiro words for a seed."""
    r = np.zeros(4, dtype=np.uint64)
    lib().ana_rng_seeded(seed & 0xFFFFFFFFFFFFFFFF, _p(r, C.c_uint64))
    return r


def rng_of(sample_seed: str) -> np.ndarray:
    """dc.rng.of: SAMPLE_SEED parsed as U64, else seed 0."""
    v = u64_read(sample_seed)
    return rng_seeded(0 if v is None else v)


class Decoder:
    """A checkpoint on a device with state for max_seqs sequences."""

    def __init__(self, path: str, device: int = 0, max_seqs: int = 1, prefill_chunk: int = 64,
                 numerics: int = EXACT_FP32):
        L = lib()
        h = C.c_void_p()
        o = _Opts(device, numerics, max_seqs, prefill_chunk)
        r = L.ana_open(path.encode(), C.byref(o), C.byref(h))
        if r != ANA_OK:
            raise AnaError(r, L.ana_error(None).decode())
        self.h = h
        cfg = _Cfg()
        step = C.c_uint64()
        self._check(L.ana_config_of(h, C.byref(cfg), C.byref(step)))
        self.config = Config(cfg.vocab, cfg.ctx, cfg.d, cfg.f, cfg.layers, cfg.heads,
                             bool(cfg.rglru), bool(cfg.qk), bool(cfg.sinks), bool(cfg.tied))
        self.step_saved = step.value
        self.max_seqs = max_seqs

    def _check(self, r: int) -> None:
        if r != ANA_OK:
            raise AnaError(r, lib().ana_error(self.h).decode())

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().ana_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def vocab(self) -> int:
        return self.config.vocab

    def reset(self, seq: int = 0) -> None:
        """dd.reset / dc.en.reset."""
        self._check(lib().ana_reset(self.h, seq))

    @staticmethod
    def _rows(s, p, t, fn: str) -> None:
        if not (p.size == t.size == s.size):
            raise ValueError(f"{fn}: {s.size} sequences, {p.size} positions, {t.size} tokens")

    @staticmethod
    def _rng(rng, n: int, fn: str):
        """The caller's n x 4 uint64 xoshiro words, advanced in place by the
        library: they must be exactly that array."""
        if not (isinstance(rng, np.ndarray) and rng.dtype == np.uint64 and rng.flags.c_contiguous
                and rng.flags.writeable and rng.size == 4 * n):
            raise ValueError(f"{fn}: rng must be a writable C-contiguous uint64 array of {4 * n} words")
        return _p(rng, C.c_uint64)

    def feed(self, seqs, pos, toks) -> None:
        """dd.feed for each listed sequence (one token each)."""
        s, p, t = _u32(seqs), _u32(pos), _u32(toks)
        self._rows(s, p, t, "feed")
        self._check(lib().ana_feed(self.h, s.size, _p(s, C.c_uint32), _p(p, C.c_uint32), _p(t, C.c_uint32)))

    def feeds(self, seq: int, pos: int, toks) -> None:
        """dd.feeds: a prompt a chunk at a time."""
        t = _u32(toks)
        self._check(lib().ana_feeds(self.h, seq, pos, _p(t, C.c_uint32), t.size))

    def feeds_n(self, seqs, pos, toks) -> None:
        """dd.feeds for several sequences at once: toks[i] into seqs[i] from
        pos[i]; each chunk step's rows share the products."""
        s, p = _u32(seqs), _u32(pos)
        ts = [_u32(t) for t in toks]
        ln = np.array([t.size for t in ts], dtype=np.uint32)
        flat = np.ascontiguousarray(np.concatenate(ts) if ts else np.zeros(0, np.uint32), dtype=np.uint32)
        if flat.size == 0:
            flat = np.zeros(1, np.uint32)
        self._check(lib().ana_feeds_n(self.h, s.size, _p(s, C.c_uint32), _p(p, C.c_uint32),
                                      _p(ln, C.c_uint32), _p(flat, C.c_uint32)))

    def score_n(self, seqs, pos, toks) -> list:
        """Evaluate.bend's window.go for several sequences: each feeds
        toks[i][:-1] from pos[i]; element t of the i-th result is
        G.lse(logits after token t) - logits[toks[i][t + 1]]."""
        s, p = _u32(seqs), _u32(pos)
        ts = [_u32(t) for t in toks]
        ln = np.array([t.size for t in ts], dtype=np.uint32)
        flat = np.ascontiguousarray(np.concatenate(ts) if ts else np.zeros(0, np.uint32), dtype=np.uint32)
        if flat.size == 0:
            flat = np.zeros(1, np.uint32)
        nce = [max(int(k) - 1, 0) for k in ln]
        out = np.zeros(max(sum(nce), 1), dtype=np.float32)
        self._check(lib().ana_score_n(self.h, s.size, _p(s, C.c_uint32), _p(p, C.c_uint32),
                                      _p(ln, C.c_uint32), _p(flat, C.c_uint32), _p(out, C.c_float)))
        res, o = [], 0
        for k in nce:
            res.append(out[o:o + k].copy())
            o += k
        return res

    def logits(self, seqs) -> np.ndarray:
        s = _u32(seqs)
        out = np.empty((s.size, self.vocab), dtype=np.float32)
        self._check(lib().ana_logits(self.h, s.size, _p(s, C.c_uint32), _p(out, C.c_float)))
        return out

    def top(self, seqs) -> np.ndarray:
        """dd.top: greedy pick on the device (vocab on a NaN max)."""
        s = _u32(seqs)
        out = np.empty(s.size, dtype=np.uint32)
        self._check(lib().ana_top(self.h, s.size, _p(s, C.c_uint32), _p(out, C.c_uint32)))
        return out

    def stats(self, seqs, toks):
        """dc.prob.of and al.stat after each sequence's last fed token: the
        token's probability, the likeliest other token and its probability."""
        s, t = _u32(seqs), _u32(toks)
        if s.size != t.size:
            raise ValueError("stats: one token per sequence")
        p = np.empty(s.size, dtype=np.float32)
        a = np.empty(s.size, dtype=np.uint32)
        pa = np.empty(s.size, dtype=np.float32)
        self._check(lib().ana_stats(self.h, s.size, _p(s, C.c_uint32), _p(t, C.c_uint32), _p(p, C.c_float),
                                    _p(a, C.c_uint32), _p(pa, C.c_float)))
        return p, a, pa

    def pick(self, seqs, st: Settings, rng: np.ndarray | None = None) -> np.ndarray:
        """S.pick on the device; rng (n x 4 uint64) advances in place."""
        s = _u32(seqs)
        out = np.empty(s.size, dtype=np.uint32)
        rp = None if rng is None else self._rng(rng, s.size, "pick")
        sc = st._c()
        self._check(lib().ana_pick(self.h, s.size, _p(s, C.c_uint32), C.byref(sc), rp, _p(out, C.c_uint32)))
        return out

    def generate(self, seqs, pos, toks, steps: int, st: Settings | None = None,
                 rng: np.ndarray | None = None) -> np.ndarray:
        """The token loop for each sequence: feed, head, pick, feed the pick."""
        s, p, t = _u32(seqs), _u32(pos), _u32(toks)
        self._rows(s, p, t, "generate")
        out = np.empty((s.size, steps), dtype=np.uint32)
        sp = C.byref(st._c()) if st is not None else None
        rp = None if rng is None else self._rng(rng, s.size, "generate")
        self._check(lib().ana_generate(self.h, s.size, _p(s, C.c_uint32), _p(p, C.c_uint32),
                                       _p(t, C.c_uint32), steps, sp, rp, _p(out, C.c_uint32)))
        return out

    KINDS = ("gemv", "head", "attn", "gla", "pick", "step")

    def prof(self, on: bool) -> None:
        """Start (and clear) or stop per-launch event timing."""
        self._check(lib().ana_prof(self.h, int(on)))

    def prof_read(self) -> dict:
        """{kind: (launches, ms, algorithmic bytes)} since prof(True)."""
        out = {}
        for k, name in enumerate(self.KINDS):
            n, ms, b = C.c_uint64(), C.c_double(), C.c_double()
            self._check(lib().ana_prof_read(self.h, k, C.byref(n), C.byref(ms), C.byref(b)))
            out[name] = (n.value, ms.value, b.value)
        return out

    def trace(self, steps: int) -> None:
        """Arm (steps >= 1) or disarm (0) the persistent decode kernel's
        phase stamps."""
        self._check(lib().ana_trace(self.h, steps))

    def trace_read(self) -> np.ndarray:
        """The last persistent launch's stamps: [steps, phases, workgroups, 4]
        ticks of the device's constant-rate clock, its low 32 bits (start,
        inputs seen, weights landed, outputs published)."""
        dims = np.zeros(3, dtype=np.uint32)
        self._check(lib().ana_trace_read(self.h, None, 0, _p(dims, C.c_uint32)))
        n = int(np.prod(dims.astype(np.int64))) * 4
        out = np.zeros(n, dtype=np.uint32)
        if n:
            self._check(lib().ana_trace_read(self.h, _p(out, C.c_uint32), n, _p(dims, C.c_uint32)))
        return out.reshape(int(dims[0]), int(dims[1]), int(dims[2]), 4)

    def state(self, seq: int, layer: int) -> np.ndarray:
        c = self.config
        if layer == c.layers:
            n = c.d
        elif c.is_softmax(layer):
            n = 2 * c.ctx * c.d
        else:
            n = c.heads * c.hd * c.hd
        out = np.empty(n, dtype=np.float32)
        self._check(lib().ana_state(self.h, seq, layer, _p(out, C.c_float), n))
        return out


def probe_reread(nbytes: int, reps: int = 20, device: int = 0) -> float:
    """ana_probe_reread: GB/s of re-reading one device buffer of nbytes."""
    g = C.c_double()
    r = lib().ana_probe_reread(device, nbytes, reps, C.byref(g))
    if r != 0:
        raise AnaError(r, f"ana_probe_reread: {nbytes} bytes")
    return g.value


def truncate_at_eos(row: np.ndarray) -> np.ndarray:
    """Generate's stop (bend/Generate.bend:31-51): the picks through the first EOS."""
    hit = np.nonzero(row == EOS)[0]
    return row if hit.size == 0 else row[: hit[0] + 1]


def window_mean(ce) -> np.float32:
    """window.mean (bend/Evaluate.bend:46-48): the F32 sum of a window's
    summands in order, over their count."""
    acc = np.float32(0.0)
    for v in np.asarray(ce, dtype=np.float32):
        acc = np.float32(acc + v)
    return np.float32(acc / np.float32(max(len(ce), 1)))


# ---------------------------------------------------------------- tokenizer

def sha256_hex(data: bytes) -> str:
    """H.sha256 (bend/Sha256.bend) in the library: 64 lowercase hex digits."""
    b = (C.c_uint8 * max(len(data), 1)).from_buffer_copy(data or b"\0")
    out = C.create_string_buffer(65)
    if lib().ana_sha256_hex(b, len(data), out) != 0:
        raise AnaError(1, "ana_sha256_hex failed")
    return out.value.decode()


class Tokenizer:
    """The fast BPE tokenizer (bend/Tokenizer.bend) through libana: ids
    0 = BOS, 1 = EOS, 2..257 the bytes, then one per merge."""

    BOS, EOS = 0, 1

    def __init__(self, path: str | None = None):
        h = C.c_void_p()
        if path is None:
            rc = lib().ana_bpe_bytes(C.byref(h))
        else:
            rc = lib().ana_bpe_open(path.encode(), C.byref(h))
        if rc != 0:
            raise AnaError(rc, f"tokenizer: cannot read a BPE artifact from {path}")
        self.h = h

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().ana_bpe_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def vocab(self) -> int:
        return int(lib().ana_bpe_vocab(self.h))

    def identity(self) -> str:
        buf = C.create_string_buffer(512)
        if lib().ana_bpe_identity(self.h, buf, 512) != 0:
            raise AnaError(1, "ana_bpe_identity failed")
        return buf.value.decode()

    def encode(self, data: bytes) -> np.ndarray:
        """Bpe.encode: the ids of a byte string (no BOS or EOS added)."""
        b = (C.c_uint8 * max(len(data), 1)).from_buffer_copy(data or b"\0")
        n = C.c_size_t()
        lib().ana_bpe_encode(self.h, b, len(data), None, 0, C.byref(n))
        out = np.zeros(max(n.value, 1), dtype=np.uint32)
        if lib().ana_bpe_encode(self.h, b, len(data), _p(out, C.c_uint32), out.size, C.byref(n)) != 0:
            raise AnaError(1, "ana_bpe_encode failed")
        return out[: n.value]

    def decode(self, ids) -> bytes:
        """Bpe.decode of each id, concatenated (BOS and EOS give no bytes)."""
        a = _u32(ids)
        a1 = a if a.size else np.zeros(1, np.uint32)
        n = C.c_size_t()
        lib().ana_bpe_decode(self.h, _p(a1, C.c_uint32), a.size, None, 0, C.byref(n))
        out = (C.c_uint8 * max(n.value, 1))()
        if lib().ana_bpe_decode(self.h, _p(a1, C.c_uint32), a.size, out, n.value, C.byref(n)) != 0:
            raise AnaError(1, "ana_bpe_decode failed")
        return bytes(out[: n.value])


# dc.candidates (bend/Decode.bend:64-66), relative to the working directory
CANDIDATES = ["weights/enwiki-fineweb-32k.bpe", "run/enwiki-fineweb-32k.bpe",
              "weights/code32k.bpe", "run/code32k.bpe", "run/enwiki-c4-32k.bpe"]
BYTE_IDENTITY = "lossless-byte-v1:bos=0:eos=1:bytes=2..257"


def find_tokenizer(want: str, pinned: str = "", candidates=None) -> Tokenizer:
    """dc.tok.of / dc.tok.btc (bend/Decode.bend:80-145,261-270): the byte
    tokenizer for its identity; else TOKENIZER_FILE (pinned) if set, which
    must match; else the first candidate whose identity matches. Failures
    carry the reference's messages."""
    if want == BYTE_IDENTITY:
        return Tokenizer(None)
    if pinned:
        try:
            t = Tokenizer(pinned)
        except AnaError:
            t = None
        if t is None or t.identity() != want:
            raise AnaError(6, "TOKENIZER_FILE identity does not match the checkpoint\n  checkpoint: " + want)
        return t
    for p in (CANDIDATES if candidates is None else candidates):
        if not os.path.exists(p):
            continue
        try:
            t = Tokenizer(p)
        except AnaError:
            continue
        if t.identity() == want:
            return t
    raise AnaError(6, "checkpoint uses BPE and no candidate tokenizer matches its identity\n  checkpoint: "
                   + want + "\n  set TOKENIZER_FILE to the matching .bpe artifact")


def read_manifest(path: str) -> dict:
    """Load.header's Manifest (bend/Checkpoint.bend:19-136) of an FTC2 file,
    through the library: every field, the doubles as the reference forms
    them in F32."""
    m = _Manifest()
    r = lib().ana_manifest_read(path.encode(), C.byref(m))
    if r != 0:
        raise AnaError(r, lib().ana_error(None).decode())
    out = {f: getattr(m, f) for f, _ in _Manifest._fields_ if f != "cfg"}
    for k in ("layout", "model_id", "tokenizer_id", "dataset_id"):
        out[k] = out[k].decode("utf-8")
    out["has_muon"] = bool(out["has_muon"])
    out["cfg"] = {f: int(getattr(m.cfg, f)) for f, _ in _Cfg._fields_}
    return out
