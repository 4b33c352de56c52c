"""Write ``reference_vectors.json``: the known-answer data the reference's own tests hold.

Reads alexandreteles/tinygrad-dx12's test sources as text (``ast``; nothing is
imported or executed) and records the literal tables, plus the exact cases whose
expected values those tests state.  Run in a container that has the reference
mounted at /root/reference; the JSON it writes is committed, so tests never read
the reference.
"""

import ast
import json
from pathlib import Path

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "reference_vectors.json"


def literal(path: Path, name: str):
    tree = ast.parse(path.read_text())
    for node in tree.body:
        if isinstance(node, ast.Assign) and any(isinstance(t, ast.Name) and t.id == name for t in node.targets):
            return ast.literal_eval(node.value), node.lineno
    raise KeyError(name)


def main() -> None:
    test_packed = REF / "test/backend/test_packed.py"
    golden, line = literal(test_packed, "GOLDEN")
    vectors = {
        "golden_positive_values": {
            "source": f"test/backend/test_packed.py:{line}",
            "values": {fmt: [float(v) for v in vals] for fmt, vals in golden.items()},
        },
        # test_packed.py:104-108: payloads 0..15 decoded by int4 / uint4
        "integer_nibbles": {
            "source": "test/backend/test_packed.py:104-108",
            "int4": list(range(8)) + list(range(-8, 0)),
            "uint4": list(range(16)),
        },
        # test_packed.py:111-115
        "scales_stay_with_k_blocks": {
            "source": "test/backend/test_packed.py:111-115",
            "data": [0x22, 0x22], "format": "fp4_e2m1", "shape": [1, 4], "scales": [[2, 7]], "block_size": 2,
            "rhs": [[1], [2], [3], [4]], "expected": [[55.0]],
        },
        # test_packed.py:127-144
        "double_block_scales": {
            "source": "test/backend/test_packed.py:127-144",
            "data": [0x22], "format": "fp4_e2m1", "shape": [1, 2],
            "scales": [[1099511627776.25, -1099511627776.0]], "block_size": 1,
            "decoded": [[1099511627776.25, -1099511627776.0]], "rhs": [[1.0], [1.0]], "expected": [[0.25]],
        },
        # test_packed.py:147-174: 17-byte pattern and the [2, 7, 11] scales around 2**31
        "large_bit_positions": {
            "source": "test/backend/test_packed.py:147-174",
            "pattern": [(i * 37 + 13) % 256 for i in range(17)],
            "scales": [2, 7, 11],
            "cases": [[fmt, kind, False] for fmt in ("uint4", "fp6_e2m3", "fp6_e3m2") for kind in ("bit", "element")]
            + [["uint4", "element", True]],
        },
        # README.md:158-172 uint4 example
        "readme_uint4": {
            "source": "README.md:158-172",
            "data": [0x21, 0x43], "shape": [2, 2], "unpacked": [[1, 2], [3, 4]],
            "column": [[1.0], [2.0]], "matmul": [[5.0], [11.0]], "vector": [1.0, 2.0], "matvec": [5.0, 11.0],
        },
        # scripts/benchmark_dtypes.py:70-74 exact {-1, 0, 1} payload codes
        "unit_codes": {
            "source": "scripts/benchmark_dtypes.py:70-74",
            "fp6_e2m3": {"-1": 40, "0": 0, "1": 8},
            "fp6_e3m2": {"-1": 44, "0": 0, "1": 12},
            "fp4_e2m1": {"-1": 10, "0": 0, "1": 2},
            "int4": {"-1": 15, "0": 0, "1": 1},
        },
        # test_linalg.py:202-218 packed integer precision
        "packed_integer_precision": {
            "source": "test/backend/test_linalg.py:202-218",
            "cases": [
                {"format": "int4", "byte": 0xF1, "dtype": "int32", "values": [16777217, 16777219], "expected": -2},
                {"format": "int4", "byte": 0xF1, "dtype": "int64", "values": [1099511627777, 1099511627779], "expected": -2},
                {"format": "uint4", "byte": 0x31, "dtype": "uint64", "values": [1099511627777, 1099511627779],
                 "expected": 4398046511114},
            ],
        },
        # test_linalg.py:173-183 wide fallback
        "wide_matrix_fallback": {
            "source": "test/backend/test_linalg.py:173-183",
            "cases": [
                {"dtype": "float64", "values": [1099511627776.25, 1.0, -1099511627776.0], "expected": 1.25},
                {"dtype": "int64", "values": [1099511627776, 7, -1099511627776], "expected": 7},
            ],
        },
        # test_linalg.py:221-230 accumulator width
        "accumulator_width": {
            "source": "test/backend/test_linalg.py:221-230",
            "cases": [{"dtype": "int8", "values": [100, 120], "acc": "int32"},
                      {"dtype": "uint8", "values": [200, 250], "acc": "uint32"}],
        },
        # test_linalg.py:119-127 fp16 inputs keep fp32 accumulation
        "fp16_accumulation": {
            "source": "test/backend/test_linalg.py:119-127",
            "matrix": [[2048.0, 1.0, -2048.0]], "vector": [1.0, 1.0, 1.0], "expected": [1.0],
        },
    }
    OUT.write_text(json.dumps(vectors, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
