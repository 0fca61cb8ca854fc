"""FTC2 checkpoints: writer, header reader and fresh parameters.

The file format is bend/Checkpoint.bend's (magic "FTC2", a Data.Binary
manifest, version 4) followed by bend/Dense/Ckpt.bend:21-34's parameter
section: a u64 count P, P big-endian f32, then the Adam step (i64) and the
first moment's count. The dense decoder reads only through the step and that
count (bend/Dense/Decode.bend:689-699, the "short read" guard), so the writer
stops there unless ``moments=True`` asks for zeroed moments as well.
"""
from __future__ import annotations

import math
import struct

import numpy as np

from .config import Config, layout

MAGIC = 1179927346  # "FTC2", bend/Checkpoint.bend:28-29
LAYOUT = "hybrid-gla-decoder-flat-parameters"
LAYOUT_VERSION = 3
MANIFEST_VERSION = 4


def _nat(n: int) -> bytes:
    """Save.nat: an Int64 below 2^32 (bend/Checkpoint.bend:196-198)."""
    return struct.pack(">Q", n)


def _string(s: str) -> bytes:
    """Save.string: Int64 character count, then UTF-8 (bend/Checkpoint.bend:232-234)."""
    return _nat(len(s)) + s.encode("utf-8")


def _double(x: float) -> bytes:
    """Save.double: decodeFloat's pair, the mantissa doubled until whole
    (tag 0, Int32) and the exponent as the Int64 -k (bend/Checkpoint.bend:236-252)."""
    x = float(np.float32(x))
    m, k = x, 0
    while k < 200 and math.floor(m) != m:
        m *= 2.0
        k += 1
    return b"\x00" + struct.pack(">i", int(m)) + struct.pack(">q", -k)


def manifest_bytes(c: Config, tokenizer_id: str = "", dataset_id: str = "synthetic", *,
                   adamw=(3.0e-4, 0.9, 0.95, 1.0e-8, 0.1, 0, 0), muon=None, clip: float = 1.0,
                   numerics: int = 0) -> bytes:
    """Save.header: magic and manifest (bend/Checkpoint.bend:254-276).
    adamw is (lr, beta1, beta2, eps, decay, warmup, total steps)."""
    out = [struct.pack(">I", MAGIC), struct.pack(">I", MANIFEST_VERSION)]
    out += [_nat(c.vocab), _nat(c.ctx), _nat(c.d), _nat(c.f), _nat(c.layers), _nat(c.heads)]
    out += [bytes([int(c.rglru)]), bytes([int(c.qk)]), bytes([int(c.sinks)]), bytes([int(c.tied)])]
    out += [_nat(c.params), _string(LAYOUT), struct.pack(">I", LAYOUT_VERSION)]
    lr, b1, b2, eps, wd, warm, total = adamw
    out += [_double(lr), _double(b1), _double(b2), _double(eps), _double(wd), _nat(warm), _nat(total)]
    out += [b"\x00"] if muon is None else [b"\x01", _double(muon)]
    out += [_string(c.model_id), _string(tokenizer_id), _string(dataset_id), _double(clip),
            bytes([numerics])]
    return b"".join(out)


def write(path: str, c: Config, params: np.ndarray, step: int = 0, tokenizer_id: str = "",
          moments: bool = False, **manifest) -> None:
    """Write an FTC2 checkpoint holding ``params`` (P float32, namedLayout
    order); ``manifest`` passes dataset_id, adamw, muon, clip, numerics to
    manifest_bytes."""
    params = np.ascontiguousarray(params, dtype=np.float32)
    if params.size != c.params:
        raise ValueError(f"params has {params.size} floats, config needs {c.params}")
    with open(path, "wb") as fp:
        fp.write(manifest_bytes(c, tokenizer_id, **manifest))
        fp.write(struct.pack(">Q", c.params))
        chunk = 1 << 24
        for i in range(0, params.size, chunk):
            fp.write(params[i:i + chunk].astype(">f4").tobytes())
        fp.write(struct.pack(">q", step))
        fp.write(struct.pack(">Q", c.params))
        if moments:
            z = np.zeros(min(chunk, c.params), dtype=">f4").tobytes()
            for _ in range(2):
                left = c.params
                while left:
                    n = min(left, chunk)
                    fp.write(z[: 4 * n])
                    left -= n
                fp.write(struct.pack(">Q", c.params))
            fp.write(b"\x00")


def read_config(path: str) -> Config:
    """The Config of an FTC2 file's manifest (bend/Checkpoint.bend:100-112)."""
    with open(path, "rb") as fp:
        head = fp.read(4 + 4 + 6 * 8 + 4)
    magic, _version = struct.unpack(">II", head[:8])
    if magic != MAGIC:
        raise ValueError("not a compact checkpoint (magic is not FTC2)")
    nums = struct.unpack(">6Q", head[8:56])
    flags = head[56:60]
    return Config(*[int(n & 0xFFFFFFFF) for n in nums], *[b != 0 for b in flags])


# -- fresh parameters --------------------------------------------------------

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _mix64(z: np.ndarray) -> np.ndarray:
    """SplitMix64's finalizer on uint64 arrays (wrapping arithmetic)."""
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def _uniform01(seed: int, idx: np.ndarray) -> np.ndarray:
    """Counter-based uniform doubles in [0, 1): SplitMix64 of seed*golden + idx."""
    with np.errstate(over="ignore"):
        base = np.uint64((seed * 0x9E3779B97F4A7C15 + 0x632BE59BD9B4E019) & 0xFFFFFFFFFFFFFFFF)
        z = _mix64(idx.astype(np.uint64) * np.uint64(0x9E3779B97F4A7C15) + base)
    return (z >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def _normal(seed: int, start: int, n: int, std: float) -> np.ndarray:
    """N(0, std^2) by Box-Muller in double from two counter streams, to f32."""
    i = np.arange(start, start + n, dtype=np.uint64)
    u1 = _uniform01(seed, np.uint64(2) * i)
    u2 = _uniform01(seed, np.uint64(2) * i + np.uint64(1))
    r = np.sqrt(-2.0 * np.log1p(-u1))
    return (std * r * np.cos(2.0 * np.pi * u2)).astype(np.float32)


def _hash_noise(idx: np.ndarray) -> np.ndarray:
    """hashNoise of bend/Train/Init.bend:24-29 in f32 steps."""
    with np.errstate(over="ignore"):
        z0 = idx.astype(np.uint64) * np.uint64(0x9E3779B97F4A7C15)
        z3 = _mix64(z0)
    hi = (z3 >> np.uint64(32)).astype(np.uint32).astype(np.float32)
    lo = (z3 & np.uint64(0xFFFFFFFF)).astype(np.uint32).astype(np.float32)
    f = hi * np.float32(4294967296.0) + lo
    return f / np.float32(9223372036854775808.0) - np.float32(1.0)


def init_params(c: Config, kind: str = "normal", seed: int = 0, std: float = 0.02,
                trained: bool = False) -> np.ndarray:
    """Fresh parameters in namedLayout order.

    kind "normal": matrices and the embedding N(0, std^2) from a counter-based
    SplitMix64 stream (the BASELINE configs' wording); "hash": the
    reference's seedless hash noise, 0.02 * hashNoise(flat index + 1)
    (bend/Train/Init.bend:17-35). Gains are 1, qk gains and sink logits 0, and
    the RG-LRU bases follow Griffin's init, sigmoid(lam)^8 uniform on
    [0.9, 0.999) (bend/Train/Init.bend:31-35).

    trained=True gives the vectors a trained checkpoint carries instead of
    their fresh values, so every use of them is exercised: RMSNorm gains
    (ra, rf, final) 1 + N(0, 0.1^2), qk-norm gains (gq, gk) N(0, 0.1^2), and
    one sink logit per head N(0, 1), each from its own counter stream of
    ``seed``.
    """
    blocks, fin = layout(c)
    p = np.empty(c.params, dtype=np.float32)
    chunk = 1 << 23

    def noise(o: int, n: int) -> None:
        for s in range(0, n, chunk):
            m = min(chunk, n - s)
            if kind == "normal":
                p[o + s:o + s + m] = _normal(seed, o + s, m, std)
            elif kind == "hash":
                idx = np.arange(o + s + 1, o + s + m + 1, dtype=np.uint64)
                p[o + s:o + s + m] = np.float32(0.02) * _hash_noise(idx)
            else:
                raise ValueError(f"unknown init kind {kind!r}")

    def lam(o: int, n: int) -> None:
        idx = np.arange(o + 1, o + n + 1, dtype=np.uint64)
        if kind == "hash":
            u01 = (_hash_noise(idx).astype(np.float64) + 1.0) / 2.0
        else:
            u01 = _uniform01(seed + 1, idx)
        u = 0.9 + 0.099 * u01
        a = u ** 0.125
        p[o:o + n] = np.log(a / (1.0 - a)).astype(np.float32)

    def vec(o: int, n: int, base: float, sd: float) -> None:
        # a trained vector: base + N(0, sd^2), indexed by its flat offset
        p[o:o + n] = base if not trained else np.float32(base) + _normal(seed + 0x7EA1, o, n, sd)

    d, f, dd = c.d, c.f, c.d * c.d
    noise(0, c.vocab * d)
    for b in blocks:
        vec(b.ra, d, 1.0, 0.1)
        noise(b.wq, 4 * dd)
        if b.gla:
            noise(b.wa, dd)
            if c.rglru:
                lam(b.lam, d)
        else:
            if c.qk:
                vec(b.gq, 2 * c.hd, 0.0, 0.1)
            if c.sinks:
                vec(b.sink, c.heads, 0.0, 1.0)
        vec(b.rf, d, 1.0, 0.1)
        noise(b.wg, 3 * f * d)
    vec(fin, d, 1.0, 0.1)
    if not c.tied:
        noise(fin + d, c.vocab * d)
    return p


def prompt(seed: int, length: int, vocab: int) -> np.ndarray:
    """A synthetic prompt: BOS (0), then length-1 ids uniform in [2, vocab)."""
    if length <= 0:
        return np.zeros(0, dtype=np.uint32)
    u = _uniform01(seed + 0x5EED, np.arange(length - 1, dtype=np.uint64))
    ids = 2 + np.floor(u * (vocab - 2)).astype(np.uint64)
    return np.concatenate([[0], ids]).astype(np.uint32)
