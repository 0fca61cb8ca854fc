import Base

# libana (include/ana.h) as Bend foreign effects, declared the way
# BulkIo.bend declares its bulk ops (/root/reference/bend/BulkIo.bend:16-93):
# a def whose body imports the C file that registers its handler
# (effs/ana.c). Bend is not installed where this file was written, so it has
# not been compiled.
#
# A context handle is a small U32 (an index into the C side's table of
# open contexts). Arrays are the caller's own Array<F32> blocks, read and
# written in place as bk.read_f32be writes its array:
# - token ids travel as F32 cells holding the id's value (ids < 2^24 are
#   exact in F32; the vocabulary is 32768);
# - an Rng (Sample.bend's four N.U64 words s0..s3, each N.U64{hi, lo})
#   travels as 8 cells: cell at + 2 i holds F32.from_bits(hi of word i) and
#   cell at + 2 i + 1 F32.from_bits(lo of word i);
# - logits and window summands come back as the F32 values themselves.
# A failed call ends the program with the library's message (err_fail), as
# a failed bulk op does.

# ana_open: the FTC2 checkpoint at path (Checkpoint.bend's format), in one
# of the numerics modes (0 exact fp32, 1 fast fp32, 2 bf16 weights), for up
# to max_seqs sequences, prefilling chunk tokens at a time (0: 64)
def ana.open(path: String, numerics: U32, max_seqs: U32, chunk: U32) -> IO(U32):
  import "./effs/ana.c"

# the Adam step the checkpoint was saved at (ana_config_of's step; the
# Model's step, as dd.load reads it)
def ana.step(h: U32) -> IO(U32):
  import "./effs/ana.c"

# dd.reset (Dense/Decode.bend:534-538): the sequence's states to zero
def ana.reset(h: U32, seq: U32) -> IO(U32):
  import "./effs/ana.c"

# dd.feed (Dense/Decode.bend:548-551): one token at pos, no head
def ana.feed(h: U32, seq: U32, pos: U32, tok: U32) -> IO(U32):
  import "./effs/ana.c"

# dd.feeds (Dense/Decode.bend:637-639): the n ids in cells x[at .. at + n)
# from pos, a chunk at a time
def ana.feeds(h: U32, seq: U32, pos: U32, x: Array<F32>, at: U32, n: U32) -> IO(Array<F32>):
  import "./effs/ana.c"

# dd.logits (Dense/Decode.bend:641-646): the head's vocab logits on the last
# fed token, into cells x[at .. at + vocab)
def ana.logits(h: U32, seq: U32, x: Array<F32>, at: U32) -> IO(Array<F32>):
  import "./effs/ana.c"

# dd.top (Dense/Decode.bend:475-484): the least index reaching the maximum
# logit, on the device; vocab when none does (a NaN maximum), where the
# caller takes the meaning's way, as dc.px.top does
def ana.top(h: U32, seq: U32) -> IO(U32):
  import "./effs/ana.c"

# S.pick (Sample.bend:246-254) with Settings{temperature, top_k, top_p}: the
# Rng's 8 cells r[at .. at + 8) are read, advanced by the draw and written
# back (untouched when greedy)
def ana.pick(h: U32, seq: U32, temperature: F32, top_k: U32, top_p: F32, r: Array<F32>, at: U32) -> IO(U32 & Array<F32>):
  import "./effs/ana.c"

# Evaluate.bend's window.go (Evaluate.bend:33-44) for one window of n ids in
# cells x[at .. at + n): its first n - 1 ids are fed from pos, and after
# each, G.lse(logits) - logits[next id] is written over cells
# x[at .. at + n - 1) (the last id's cell keeps its value); window.mean is
# then the in-order F32 sum of those n - 1 cells over n - 1
def ana.score(h: U32, seq: U32, pos: U32, x: Array<F32>, at: U32, n: U32) -> IO(Array<F32>):
  import "./effs/ana.c"
