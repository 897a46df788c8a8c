"""Writes the golden fixtures under tests/golden/.

  kat_quantize.json -- known answers for QuantizedTensor.quantize
      (Engine/kotensor/src/main/kotlin/QuantizedTensor.kt:256-324). Every expected
      value below was derived by hand from IEEE-754 binary32 arithmetic and the JDK
      contract of Math.round (nearest, ties toward +inf, saturating), not computed
      by the oracle. Two cases are found by a numpy search for inputs where
      multiplying by the reciprocal and dividing round to different integers; their
      expected values come from numpy's IEEE float32 product/quotient and exact
      rounding in float64.
  fixtures.npz -- small regression vectors produced by the oracle (inputs,
      packed bytes, scales, zeros, and matmul outputs for fixed activations).

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

SUB = float(np.float32(2.0) ** -149)  # smallest subnormal, 2^-149


def f32_bits(x: float) -> int:
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def hand_kats() -> list[dict]:
    kats = []
    # INT8: maxAbs = 127 -> scale = 1, inverse = 1, q = Math.round(x).
    kats.append({
        "name": "int8_ties_scale_one", "bits": 8, "group": 16, "rows": 12, "columns": 1,
        "data": [127.0, 2.5, -2.5, 0.5, -0.5, 0.49999997, -126.5, 126.5, 1.5, -1.5, 0.0, -0.0],
        "qdata": [127, 3, -2, 1, 0, 0, -126, 127, 2, -1, 0, 0],
        "scales": [1.0], "zeros": None, "status": 0,
    })
    # INT8 all zero: scale 1, q 0.
    kats.append({
        "name": "int8_all_zero", "bits": 8, "group": 4, "rows": 4, "columns": 2,
        "data": [0.0] * 8, "qdata": [0] * 8, "scales": [1.0, 1.0], "zeros": None, "status": 0,
    })
    # INT8 subnormal maxAbs = 20*2^-149: 20/127 * 2^-149 rounds to 0 -> scale 0,
    # inverse +inf, x*inverse = +-inf -> Math.round saturates -> clamp to +-127.
    kats.append({
        "name": "int8_scale_underflows_to_zero", "bits": 8, "group": 2, "rows": 2, "columns": 1,
        "data": [20 * SUB, -20 * SUB], "qdata": [127, -127], "scales": [0.0], "zeros": None, "status": 0,
    })
    # INT8 with an infinity: maxAbs = inf -> scale inf -> inverse 0 -> inf * 0 = NaN -> throws.
    kats.append({
        "name": "int8_inf_is_nan_error", "bits": 8, "group": 2, "rows": 2, "columns": 1,
        "data": [float("inf"), 1.0], "status": -3,
    })
    # NaN in the data is skipped by the max but rejected by roundToInt.
    kats.append({
        "name": "int8_nan_error", "bits": 8, "group": 2, "rows": 2, "columns": 1,
        "data": [float("nan"), 1.0], "status": -3,
    })
    # INT4: min -7.5, max 7.5 -> range 15, scale 1, zero = round(7.5) = 8, q = round(x) + 8.
    kats.append({
        "name": "int4_ties_scale_one", "bits": 4, "group": 16, "rows": 11, "columns": 1,
        "data": [-7.5, 7.5, 0.0, 1.5, -1.5, 2.5, -2.5, 7.0, -7.0, 0.5, -0.5],
        # column 0 < half = 1 -> low nibble of byte r
        "qdata": [1, 15, 8, 10, 7, 11, 6, 15, 1, 9, 8],
        "scales": [1.0], "zeros": [8], "status": 0,
    })
    # Split-half packing, N = 5 (half = 3, pad nibble in byte 2), two rows, one group:
    #   c0 [-7.5, 7.5]  scale 1 zero 8 q [1, 15]
    #   c1 [3, 15]      min clamps to 0: scale 1 zero 0 q [3, 15]
    #   c2 [0, 15]      scale 1 zero 0 q [0, 15]
    #   c3 [-3.5, 11.5] scale 1 zero round(3.5)=4 q [round(-3.5)+4=1, 16->15]
    #   c4 [7.5, -7.5]  scale 1 zero 8 q [15, 1]
    # byte c (c < 3) = q(c) | q(c+3) << 4; byte 2's high nibble is the pad (0).
    kats.append({
        "name": "int4_split_half_odd_width", "bits": 4, "group": 2, "rows": 2, "columns": 5,
        "data": [-7.5, 3.0, 0.0, -3.5, 7.5,
                 7.5, 15.0, 15.0, 11.5, -7.5],
        "qdata": [0x11, 0xF3, 0x00,
                  0xFF, 0x1F, 0x0F],
        "scales": [1.0, 1.0, 1.0, 1.0, 1.0], "zeros": [8, 0, 0, 4, 8], "status": 0,
    })
    # INT4 all positive (min clamps to 0) and all negative (max clamps to 0), g = 3.
    kats.append({
        "name": "int4_one_signed_groups", "bits": 4, "group": 3, "rows": 3, "columns": 2,
        "data": [1.0, -15.0,
                 2.0, -3.0,
                 15.0, -1.0],
        # c0: scale 1 zero 0 -> q 1, 2, 15; c1: scale 1 zero 15 -> q 0, 12, 14.
        # half = 1: byte r = q(r, c0) | q(r, c1) << 4
        "qdata": [0x01, 0xC2, 0xEF],
        "scales": [1.0, 1.0], "zeros": [0, 15], "status": 0,
    })
    # INT4 subnormal range: c = [20, -20] * 2^-149, range 40*2^-149, scale = 40/15 -> 3*2^-149,
    # zero = round(20/3 = 6.67) = 7, inverse = 2^149/3 overflows to +inf, x*inf = +-inf,
    # Math.round saturates to +-2^31 - (0|1), Kotlin's Int addition of 7 wraps the
    # positive case to a negative value, so both clamp to 0.
    kats.append({
        "name": "int4_inverse_overflow_wraps", "bits": 4, "group": 2, "rows": 2, "columns": 1,
        "data": [20 * SUB, -20 * SUB], "qdata": [0, 0], "scales": [3 * SUB], "zeros": [7], "status": 0,
    })
    # INT4 range overflow: max - min = +inf -> scale inf, zero = round(3e38/inf = 0) = 0,
    # inverse 0, q = round(x*0) + 0 = 0.
    kats.append({
        "name": "int4_range_overflow", "bits": 4, "group": 2, "rows": 2, "columns": 1,
        "data": [3.0e38, -3.0e38], "qdata": [0, 0], "scales": [float("inf")], "zeros": [0], "status": 0,
    })
    # INT4 tiny positive range with a zero element: range = 2^-149, range/15 rounds to 0
    # -> scale 0 -> zero = round(-0/0 = NaN) -> throws.
    kats.append({
        "name": "int4_zero_scale_nan_error", "bits": 4, "group": 2, "rows": 2, "columns": 1,
        "data": [SUB, 0.0], "status": -3,
    })
    return kats


def java_round_exact(p: np.ndarray) -> np.ndarray:
    return np.floor(p.astype(np.float64) + 0.5).astype(np.int64)


def search_kats(seed: int = 12345) -> list[dict]:
    """Cases where reciprocal-multiply and division give different integers."""
    rng = np.random.default_rng(seed)
    out = []
    # symmetric: q = round(x * (1 / (maxAbs / 127))) versus round(x / (maxAbs / 127))
    with np.errstate(all="ignore"):
        for _ in range(200):
            mx = rng.uniform(0.5, 2.0, 1 << 20).astype(np.float32)
            x = (rng.uniform(-1.0, 1.0, 1 << 20).astype(np.float32) * mx).astype(np.float32)
            scale = (mx / np.float32(127.0)).astype(np.float32)
            inv = (np.float32(1.0) / scale).astype(np.float32)
            a = java_round_exact((x * inv).astype(np.float32))
            b = java_round_exact((x / scale).astype(np.float32))
            hit = np.nonzero(a != b)[0]
            if hit.size:
                i = int(hit[0])
                out.append({
                    "name": "int8_reciprocal_not_division", "bits": 8, "group": 2, "rows": 2, "columns": 1,
                    "data": [float(mx[i]), float(x[i])],
                    "qdata": [127, int(a[i])], "scales": [float(scale[i])], "zeros": None, "status": 0,
                    "division_would_give": int(b[i]),
                })
                break
        # asymmetric zero point: zero = round(-min / scale) (a true division)
        for _ in range(200):
            mn = -rng.uniform(0.1, 2.0, 1 << 20).astype(np.float32)
            mx = rng.uniform(0.1, 2.0, 1 << 20).astype(np.float32)
            scale = ((mx - mn) / np.float32(15.0)).astype(np.float32)
            z_div = java_round_exact((-mn / scale).astype(np.float32))
            z_mul = java_round_exact((-mn * (np.float32(1.0) / scale)).astype(np.float32))
            hit = np.nonzero(z_div != z_mul)[0]
            if hit.size:
                i = int(hit[0])
                s = scale[i]
                inv = np.float32(1.0) / s
                qs = [int(np.clip(java_round_exact(np.array([v * inv], dtype=np.float32))[0] + z_div[i], 0, 15))
                      for v in (mn[i], mx[i])]
                out.append({
                    "name": "int4_zero_is_a_division", "bits": 4, "group": 2, "rows": 2, "columns": 1,
                    "data": [float(mn[i]), float(mx[i])],
                    "qdata": qs, "scales": [float(s)], "zeros": [int(z_div[i])], "status": 0,
                    "multiplication_would_give": int(z_mul[i]),
                })
                break
    return out


def oracle_fixtures() -> dict[str, np.ndarray]:
    import oracle

    oracle.build()
    rng = np.random.default_rng(2024)
    cases = [
        ("q8_100x37_g64", 100, 37, 8, 64),
        ("q4_100x37_g32", 100, 37, 4, 32),
        ("q4_70x9_g64", 70, 9, 4, 64),
        ("q8_2x17_g64", 2, 17, 8, 64),
        ("q4_2x17_g64", 2, 17, 4, 64),
        ("q4_130x64_g16", 130, 64, 4, 16),
        ("q8_96x40_g1000", 96, 40, 8, 1000),
    ]
    arrays: dict[str, np.ndarray] = {}
    for name, k, n, bits, g in cases:
        w = ((rng.random((k, n), dtype=np.float32) - 0.5) * 0.2).astype(np.float32)
        st, qt = oracle.quantize(w, bits, g)
        assert st == 0
        x = (rng.random((3, k), dtype=np.float32) - 0.5).astype(np.float32)
        y3 = oracle.multiply_quantized(x, qt, 3)
        y1 = oracle.multiply_quantized(x[:1], qt, 1)
        arrays[f"{name}.data"] = w
        arrays[f"{name}.qdata"] = qt.qdata
        arrays[f"{name}.scales"] = qt.scales
        if qt.zeros is not None:
            arrays[f"{name}.zeros"] = qt.zeros
        arrays[f"{name}.x"] = x
        arrays[f"{name}.y3"] = y3
        arrays[f"{name}.y1"] = y1
        arrays[f"{name}.meta"] = np.array([k, n, bits, g], dtype=np.int32)
    return arrays


def main() -> None:
    kats = hand_kats() + search_kats()
    for kat in kats:
        kat["data_bits"] = [f32_bits(v) for v in kat["data"]]
        if kat.get("scales") is not None:
            kat["scales_bits"] = [f32_bits(v) for v in kat["scales"]]
    (HERE / "kat_quantize.json").write_text(json.dumps(kats, indent=1) + "\n")
    np.savez_compressed(HERE / "fixtures.npz", **oracle_fixtures())
    print(f"wrote {len(kats)} known answers and the oracle fixtures")


if __name__ == "__main__":
    main()
