"""Writes tests/golden/golden.json from closed forms and the oracle.

The reference (alavicka/pollux) ships no tests, fixtures or golden vectors, so
the committed fixtures are: closed-form values derived by hand from the
reference's code (fingerprint, first/last codebook rows, a hand-packed group),
and SHA-256 digests of the codebook tables produced by the oracle restatement
(oracle/codebook.py), which tests then require the product's independent C++
generator to reproduce.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import codebook as cb  # noqa: E402


def main() -> None:
    f32 = cb.codebook_f32()
    out = {
        "codebook_sha256": {
            "int8_raw": hashlib.sha256(cb.codebook_int8().tobytes()).hexdigest(),
            "fp32": hashlib.sha256(f32.tobytes()).hexdigest(),
            "bf16_bits": hashlib.sha256(cb.bf16_round_bits(f32).tobytes()).hexdigest(),
            "fp16": hashlib.sha256(cb.codebook_f16().tobytes()).hexdigest(),
        },
        # castor.py:263-266 closed form: rows 0..3 are 0, (-4,-4,0..), (-4,0,-4,0..), (-4,0,0,-4,..)
        # times fp32(1/sqrt 8); 4 * 0x3EB504F3 = 0x3FB504F3 = 1.4142135381698608
        "fingerprint": [0.0] * 4
        + [-1.4142135381698608, -1.4142135381698608, 0.0, 0.0]
        + [-1.4142135381698608, 0.0, -1.4142135381698608, 0.0]
        + [-1.4142135381698608, 0.0, 0.0, -1.4142135381698608],
        "codebook_rows": {
            "1": [-4, -4] + [0] * 22,
            "2": [-4, 0, -4] + [0] * 21,
            "3": [-4, 0, 0, -4] + [0] * 20,
            "196560": [4, 4] + [0] * 22,
        },
        # 18-bit fields 0 | 1 | 196560 (0b101111111111010000) | 262143 concatenated
        # big-endian: 00 00 00 00 1B FF 43 FF FF (derived by hand, castor.py:237-245)
        "pack_vectors": [
            {"indices": [0, 1, 196560, 262143], "bytes": "000000001bff43ffff"},
            {"indices": [262143, 0, 0, 0], "bytes": "ffffc0000000000000"},
            {"indices": [5], "bytes": "000140000000000000"},
        ],
        "golay_weight_distribution": {"0": 1, "8": 759, "12": 2576, "16": 759, "24": 1},
        "type_counts": {"type1": 1104, "type2": 97152, "type3": 98304},
        "type3_off_lattice": 49152,
        "constants_f32_hex": {
            "leech_scale": "3eb504f3",
            "s_lattice": "3f3504f3",
            "c_sq_norm": "407fffff",
            "eps": "322bcc77",
            "sqrt12": "405db3d7",
        },
    }
    dst = Path(__file__).with_name("golden.json")
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {dst}")


if __name__ == "__main__":
    main()
