"""Writes tests/golden/reference_vectors.json: the known answers the
reference's own tests hold for this path, as data.

- bend/tests/num.bend:4-11 (expected lines in bend/tests/Checks.bend:436):
  U64 mul, rotl 45, shr 30, add with carry, decimal read, f32 from bits.
- bend/tests/decode-dense.bend:199-220: greedy's tie vectors; the expected
  pick is the least index holding the maximum.
- bend/tests/decode-dense.bend:24-33 and bend/tests/prefill-dense.bend:29-37:
  the token window (95 byte tokens from an LCG walk at seed 7, then 0).
- bend/tests/prefill-dense.bend:10-25,166-182: the six chunked-prefill runs
  (tokens, steps before, chunk 16, ctx 64).
"""
import json
import os


def window(n, s):
    out = []
    for _ in range(n):
        out.append(2 + ((s >> 16) & 255))
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
    return out + [0]


def main():
    v = {
        "num_kats": {
            "mul": {"a": [305419896, 2596069104], "b": [4275878552, 1985229328], "hex": "236d88fe5618cf00"},
            "rotl45": {"a": [305419896, 2596069104], "hex": "9bde02468acf1357"},
            "shr30": {"a": [305419896, 2596069104], "hex": "0000000048d159e2"},
            "add": {"a": [4294967295, 4294967295], "b": [0, 2], "hex": "0000000000000001"},
            "read": {"s": "18446744073709551615", "hex": "ffffffffffffffff"},
            "f32_from_bits": {"bytes": [63, 192, 0, 0], "value": 1.5},
        },
        "ties": [[1.0, 3.0, 3.0, 2.0], [0.0, 0.0, 0.0, 0.0], [-1.0, -5.0, -1.0, -2.0],
                 [2.0, 1.0, 0.0, 7.0], ["-0.0", 0.0, -3.0, 0.0]],
        "tie_picks": [1, 0, 0, 3, 0],
        "window": window(95, 7),
        "prefill_runs": [
            {"name": "96 from 0: 6 chunks", "pre": 0, "n": 96},
            {"name": "95 from 0: 5 chunks and one of 15", "pre": 0, "n": 95},
            {"name": "40 from 0: 2 chunks and one of 8", "pre": 0, "n": 40},
            {"name": "50 from 0: 3 chunks and 2 steps", "pre": 0, "n": 50},
            {"name": "96 from 5: 5 steps, 5 chunks and one of 11", "pre": 5, "n": 96},
            {"name": "67 from 5: 5 steps, 3 chunks and one of 14", "pre": 5, "n": 67},
        ],
        "prefill_chunk": 16,
    }
    here = os.path.dirname(os.path.abspath(__file__))
    with open(os.path.join(here, "reference_vectors.json"), "w") as f:
        json.dump(v, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
