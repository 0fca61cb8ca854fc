"""Model configuration, parameter count, identity and parameter layout.

Restates bend/Config.bend (the record, the hybrid rule, ``params``,
``model_id``, presets) and the namedLayout offsets of
bend/Dense/Layout.bend:627-686, which are the FTC2 parameter vector's order.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Config:
    """bend/Config.bend:7-10 (field order is the FTC2 manifest's)."""

    vocab: int
    ctx: int
    d: int
    f: int
    layers: int
    heads: int
    rglru: bool
    qk: bool
    sinks: bool
    tied: bool = True

    @property
    def hd(self) -> int:
        return self.d // self.heads

    def is_softmax(self, i: int) -> bool:
        """Layer i is softmax exactly when i mod 4 = 3 (bend/Config.bend:213-227)."""
        return i % 4 == 3

    @property
    def softmax_layers(self) -> int:
        return self.layers // 4

    @property
    def gla_layers(self) -> int:
        return self.layers - self.softmax_layers

    @property
    def params(self) -> int:
        """Config.params, term for term (bend/Config.bend:243-253)."""
        d, f, v = self.d, self.f, self.vocab
        p = v * d + self.layers * (4 * d * d + 3 * f * d + 2 * d) + self.gla_layers * d * d
        if self.rglru:
            p += self.gla_layers * d
        if self.qk:
            p += self.softmax_layers * 2 * self.hd
        if self.sinks:
            p += self.softmax_layers * self.heads
        p += d
        if not self.tied:
            p += v * d
        return p

    def show(self) -> str:
        """Haskell's derived Show of the record (bend/Config.bend:259-274)."""
        b = lambda x: "True" if x else "False"  # noqa: E731
        return (
            f"Config {{vocabSize = {self.vocab}, contextSize = {self.ctx}, modelDim = {self.d}, "
            f"ffDim = {self.f}, layerCount = {self.layers}, headCount = {self.heads}, "
            f"gateKind = {'GateRgLru' if self.rglru else 'GateSigmoid'}, qkNorm = {b(self.qk)}, "
            f"headSinks = {b(self.sinks)}, tiedHead = {b(self.tied)}}}"
        )

    @property
    def model_id(self) -> str:
        """bend/Config.bend:276-277."""
        return "formal-transformer-futhark-hybrid-gla-v3:" + self.show()


@dataclass(frozen=True)
class Block:
    """One layer's parameter offsets (BP of bend/Dense/Layout.bend:99-100)."""

    gla: bool
    ra: int
    wq: int
    wk: int
    wv: int
    wo: int
    wa: int
    lam: int
    gq: int
    gk: int
    sink: int
    rf: int
    wg: int
    wu: int
    wd: int
    end: int


def layout(c: Config) -> tuple[list[Block], int]:
    """BP.list and blocks.end (bend/Dense/Layout.bend:627-686): the blocks and
    the offset of the final norm's gains."""
    d, f, dd = c.d, c.f, c.d * c.d
    o = c.vocab * d
    out = []
    for i in range(c.layers):
        q = o + d
        if not c.is_softmax(i):
            lam = q + 5 * dd
            rf = lam + (d if c.rglru else 0)
            wg = rf + d
            b = Block(True, o, q, q + dd, q + 2 * dd, q + 3 * dd, q + 4 * dd, lam, 0, 0, 0, rf,
                      wg, wg + f * d, wg + 2 * f * d, wg + 3 * f * d)
        else:
            gq = q + 4 * dd
            gk = gq + (c.hd if c.qk else 0)
            sink = gk + (c.hd if c.qk else 0)
            rf = sink + (c.heads if c.sinks else 0)
            wg = rf + d
            b = Block(False, o, q, q + dd, q + 2 * dd, q + 3 * dd, 0, 0, gq, gk, sink, rf,
                      wg, wg + f * d, wg + 2 * f * d, wg + 3 * f * d)
        out.append(b)
        o = b.end
    return out, o


# Presets (bend/Config.bend:280-305) and the benchmark's configs.
SMALL4_V3 = Config(258, 64, 64, 192, 4, 4, True, True, True)
SMALL4_NOARMS = Config(258, 64, 64, 192, 4, 4, False, False, False)
TINY = Config(258, 16, 16, 48, 1, 2, False, False, False)
BPE100M_V3 = Config(32768, 256, 768, 2048, 12, 12, True, True, True)
FP100M = Config(32768, 2048, 768, 2048, 12, 12, True, True, True)
# v1 (d 256, f 1024, 4 layers, 4 heads, ctx 256), v2 (the
# 115M at ctx 256 with sigmoid gates, no qk-norm, no sinks)
V1 = Config(32768, 256, 256, 1024, 4, 4, False, False, False)
V2 = Config(32768, 256, 768, 2048, 12, 12, False, False, False)
# v2 as BASELINE.json writes it (MLP 3072: 143,739,648 parameters, not the
# reference's 115M, whose MLP is 2048)
V2_F3072 = Config(32768, 256, 768, 3072, 12, 12, False, False, False)
