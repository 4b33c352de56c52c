"""Write ``oracle_fixtures.npz``: seeded oracle inputs/outputs pinned as a regression fixture.

Run from the repository root: ``python tests/golden/make_oracle_fixtures.py``.
"""

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
import packed_oracle as O  # noqa: E402


def main() -> None:
    rng = np.random.default_rng(0)
    out = {}
    for fmt in ("int4", "fp4_e2m1", "fp6_e2m3", "fp6_e3m2"):
        n, k = 8, 128
        codes = rng.integers(0, 1 << O.bits_of(fmt), (n, k)).astype(np.uint8)
        data = O.pack_codes(codes, O.bits_of(fmt))
        if fmt == "int4":
            scales = rng.uniform(0.005, 0.02, (n, k // 32)).astype(np.float16)
            deq = O.unpack(data, fmt, (n, k), scales.astype(np.float32), 32)
        else:
            scales = (127 + rng.integers(-4, 3, (n, k // 32))).astype(np.uint8)
            deq = O.unpack(data, fmt, (n, k), O.e8m0_decode(scales), 32)
        out.update({f"{fmt}_data": data, f"{fmt}_scales": scales, f"{fmt}_shape": np.array([n, k]), f"{fmt}_deq": deq})
    x = rng.standard_normal((4, 96)).astype(np.float32)
    codes, e = O.quantize_mx(x, "fp4_e2m1", 32)
    out.update({"quant_x": x, "quant_codes": codes, "quant_e": e})
    path = Path(__file__).resolve().parent / "oracle_fixtures.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
