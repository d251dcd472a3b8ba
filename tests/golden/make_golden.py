"""Write tests/golden/reference_fixtures.json from gollek's own GGUF runtime tests.

Each fixture is data: the block bytes a reference test writes, the input
vector it uses and the outputs it asserts.  Expected values are the closed
forms the reference tests state (asserted there with tolerance 0.0) or, for
the tests that compare against an independent scalar reference at 1e-3, that
reference's own float32 formula evaluated on the same inputs.  TST/ abbreviates
runner/gguf/gollek-gguf-core/src/test/java/tech/kayys/gollek/gguf/runtime/.

Run: python tests/golden/make_golden.py  (rewrites the JSON next to it).
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "reference_fixtures.json"
Q4_0, Q8_0, Q4_K = 2, 8, 12


def bits(values) -> list[int]:
    return [int(v) for v in np.asarray(values, dtype=np.float32).view(np.uint32)]


def le16(v: int) -> list[int]:
    return [v & 0xFF, (v >> 8) & 0xFF]


# ---- block writers (restating the reference fixture helpers) -------------

def q4k_simple_block() -> list[int]:
    """TST/GgufQ4Fx.java:13-24: d=1, dmin=0, scales {1,1,1,1,0,0,0,0,1,1,1,1},
    all quant bytes 0x21."""
    return le16(0x3C00) + le16(0) + [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1] + [0x21] * 128


def q4k_all_scales_mins_block() -> list[int]:
    """TST/GgufQ4Fx.java:26-37: d=1, dmin=0.5, sc=1 and m=2 for all eight."""
    return le16(0x3C00) + le16(0x3800) + [1, 1, 1, 1, 2, 2, 2, 2, 0x21, 0x21, 0x21, 0x21] + [0x21] * 128


def q4k_lane_quants(block: list[int]) -> list[int]:
    """TST/GgufQ4CalcFx.java:10-14: byte i = (i & 15) | ((15 - (i & 15)) << 4)."""
    return block[:16] + [(i & 15) | ((15 - (i & 15)) << 4) for i in range(128)]


def q4k_lane_row(has_mins: bool) -> list[float]:
    """TST/GgufQ4CalcFx.java:28-48."""
    row = [0.0] * 256
    for sb in range(0, 256, 64):
        base = (sb // 64) * 32
        for i in range(32):
            low = (base + i) & 15
            high = 15 - ((base + i) & 15)
            row[sb + i] = low - 1.0 if has_mins else float(low)
            row[sb + 32 + i] = high - 1.0 if has_mins else float(high)
    return row


def q4_0_block(scale: int, packed: int) -> list[int]:
    """TST/GgufQ32Q4Fx.java:17-20 + :57-61."""
    return le16(scale) + [packed] * 16


def q4_0_lane_block(scale: int) -> list[int]:
    """TST/GgufQ32Q4Fx.java:22-25 with TST/GgufNibFx.java:13-25."""
    return le16(scale) + [((i & 15) | ((15 - i) << 4)) & 0xFF for i in range(16)]


def q8_block(scale: int, quant: int) -> list[int]:
    """TST/GgufQ8Fx.java:19-24."""
    return le16(scale) + [quant & 0xFF] * 32


def q8_ramp_block(scale: int, start: int) -> list[int]:
    """TST/GgufQ8Fx.java:26-31."""
    return le16(scale) + [((start + i) if start < 0 else (start - i)) & 0xFF for i in range(32)]


def q8_pattern_block(scale: int, seed: int) -> list[int]:
    """TST/GgufQ8RawTest.java:363-366 with q8Pattern = (byte)(seed + 41 i) (:410-412)."""
    return le16(scale) + [(seed + 41 * i) & 0xFF for i in range(32)]


def q5k_lane_block(has_mins: bool) -> list[int]:
    """GgufQ5LaneFx.writeNoMinBlock / writeMinBlock (TST/GgufQ5LaneFx.java:13-24,
    TST/GgufQ5Fx.java:13-55, TST/GgufQ5CalcFx.java:10-17)."""
    b = [0] * 176
    if has_mins:  # writeBlockWithMin(scale 2, min 1): d = dmin = 1.0
        b[0:2], b[2:4] = le16(0x3C00), le16(0x3C00)
        for i in range(4):
            b[4 + i], b[8 + i], b[12 + i] = 2, 1, (1 << 4) | 2
    else:         # writeBlock: d = 1.0, dmin = 0, scale codes 1
        b[0:2], b[2:4] = le16(0x3C00), le16(0)
        b[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
    for i in range(32):
        b[16 + i] = (i * 73 + 0x5A) & 0xFF
    for i in range(128):
        lo = i & 0x0F
        b[48 + i] = lo | ((15 - lo) << 4)
    return b


def q5k_lane_row(has_mins: bool) -> list[float]:
    """GgufQ5CalcFx.expectedRow (:27-66)."""
    row = [0.0] * 256
    for sb in range(0, 256, 64):
        qb = (sb // 64) * 32
        sl, shh = sb // 32, sb // 32 + 1
        for i in range(32):
            hb = (i * 73 + 0x5A) & 0xFF
            lo = ((qb + i) & 0x0F) + (((hb >> sl) & 1) << 4)
            hi = (15 - ((qb + i) & 0x0F)) + (((hb >> shh) & 1) << 4)
            row[sb + i] = 2.0 * lo - 1.0 if has_mins else float(lo)
            row[sb + 32 + i] = 2.0 * hi - 1.0 if has_mins else float(hi)
    return row


def q6k_lane_block() -> list[int]:
    """GgufQ6Fx.writeLaneOrderBlock (TST/GgufQ6Fx.java:26-38)."""
    b = [0] * 210
    for i in range(128):
        lo = i & 0x0F
        b[i] = lo | ((15 - lo) << 4)
    for i in range(64):
        b[128 + i] = (i * 53 + 0xA7) & 0xFF
    for i in range(16):
        b[192 + i] = 1
    b[208:210] = le16(0x3C00)
    return b


def q6k_lane_row() -> list[float]:
    """GgufQ6LaneFx.expectedRow (TST/GgufQ6LaneFx.java:30-48)."""
    row = [0.0] * 256
    for sb in range(0, 256, 128):
        lb, hbase = (sb // 128) * 64, (sb // 128) * 32
        for i in range(32):
            a = q6k_lane_block()[lb + i]
            bb = q6k_lane_block()[lb + 32 + i]
            hb = q6k_lane_block()[128 + hbase + i]
            row[sb + i] = float(((a & 0x0F) | ((hb & 3) << 4)) - 32)
            row[sb + 32 + i] = float(((bb & 0x0F) | (((hb >> 2) & 3) << 4)) - 32)
            row[sb + 64 + i] = float(((a >> 4) | (((hb >> 4) & 3) << 4)) - 32)
            row[sb + 96 + i] = float(((bb >> 4) | (((hb >> 6) & 3) << 4)) - 32)
    return row


def ones(n: int) -> list[float]:
    return [1.0] * n


def ramp(n: int) -> list[float]:
    return [i + 1.0 for i in range(n)]


def fixtures() -> list[dict]:
    fx: list[dict] = []

    def add(name, source, type_id, cols, rows, data, vector=None, expected_dequant=None,
            expected_matvec=None, row_count=None, tolerance=0.0, vector_offset=0):
        fx.append({
            "name": name, "source": source, "type_id": type_id, "cols": cols, "rows": rows,
            "data_hex": bytes(data).hex(),
            "vector": vector, "vector_offset": vector_offset,
            "expected_dequant_bits": [bits(r) for r in expected_dequant] if expected_dequant else None,
            "expected_matvec": expected_matvec,
            "row_count": rows if row_count is None else row_count,
            "tolerance": tolerance,
        })

    simple_row = ([1.0] * 32 + [2.0] * 32) * 4
    add("q4k_simple_block", "TST/GgufQ4KTest.java:18-49", Q4_K, 256, 1, q4k_simple_block(),
        vector=ones(256), expected_dequant=[simple_row], expected_matvec=[384.0])

    for has_mins in (False, True):
        blk = q4k_lane_quants(q4k_all_scales_mins_block() if has_mins else q4k_simple_block())
        row = q4k_lane_row(has_mins)
        dot = float(sum(np.float64(a) * b for a, b in zip(row, ramp(256))))
        assert abs(dot) < 2 ** 24 and dot == int(dot)  # exact in float32
        add(f"q4k_lane_order_{'min' if has_mins else 'nomin'}",
            "TST/GgufQ4KRawTest.java:21-68 (TST/GgufQ4CalcFx.java:16-48)", Q4_K, 256, 1, blk,
            vector=ramp(256), expected_dequant=[row], expected_matvec=[dot])

    mixed = q4k_simple_block()
    mixed[2:4] = le16(0x7E00)  # dmin = NaN, every min code zero
    add("q4k_mixed_nan_dmin_zero_min_codes", "TST/GgufQ4KMixTest.java:21-45", Q4_K, 256, 2,
        mixed + q4k_all_scales_mins_block(), vector=ones(256),
        expected_dequant=[simple_row, ([0.0] * 32 + [1.0] * 32) * 4],
        expected_matvec=[384.0, 128.0])

    add("q4k_zero_min_codes_nan_dmin_row", "TST/GgufRawKTest.java:57-88", Q4_K, 256, 1, mixed,
        vector=ones(256), expected_dequant=[simple_row], expected_matvec=[384.0])

    # TST/GgufQ4KRawTest.java:119-167: 5 rows x 5 blocks, unrolled rows + tail.
    for has_mins in (False, True):
        blk = q4k_lane_quants(q4k_all_scales_mins_block() if has_mins else q4k_simple_block())
        data = blk * 25
        vec = [np.float32((i % 41 - 20) * np.float32(0.017578125)) for i in range(5 * 256)]
        row = q4k_lane_row(has_mins) * 5
        exp = float(np.dot(np.asarray(row, np.float64), np.asarray(vec, np.float64)))
        add(f"q4k_rows5_blocks5_{'min' if has_mins else 'nomin'}",
            "TST/GgufQ4KRawTest.java:119-167", Q4_K, 5 * 256, 5, data,
            vector=[float(v) for v in vec], expected_dequant=[row] * 5,
            expected_matvec=[exp] * 5, tolerance=1e-3)

    add("q4_0_two_rows", "TST/GgufQ32Test.java:17-42", Q4_0, 32, 2,
        q4_0_block(0x3C00, 0x98) + q4_0_block(0x3C00, 0xA9), vector=ones(32),
        expected_dequant=[[0.0] * 16 + [1.0] * 16, [1.0] * 16 + [2.0] * 16],
        expected_matvec=[16.0, 48.0])

    lane_row = [float((i & 15) - 8) for i in range(16)] + [float((15 - i) - 8) for i in range(16)]
    add("q4_0_lane_order", "TST/GgufQ32Q4LaneTest.java:24-41", Q4_0, 32, 1, q4_0_lane_block(0x3C00),
        vector=ramp(32), expected_dequant=[lane_row], expected_matvec=[-264.0])

    # Signed zero: the reference adds +0.0f, so (8 - 8) * d with d = -1 is +0.0.
    add("q4_0_negative_scale_zero_nibbles", "RT/GgufBlockDequantizer.java:412-413", Q4_0, 32, 1,
        q4_0_block(0xBC00, 0x88), vector=ones(32), expected_dequant=[[0.0] * 32],
        expected_matvec=[0.0])

    add("q8_0_two_rows", "TST/GgufQ8Test.java:22-60", Q8_0, 32, 2,
        q8_block(0x3C00, 1) + q8_block(0x3C00, 2), vector=ones(32),
        expected_dequant=[[1.0] * 32, [2.0] * 32], expected_matvec=[32.0, 64.0])

    add("q8_0_signed_lane_order", "TST/GgufQ8RawTest.java:81-104", Q8_0, 32, 2,
        q8_ramp_block(0x3C00, -16) + q8_ramp_block(0x3C00, 16), vector=ramp(32),
        expected_dequant=[[float(-16 + i) for i in range(32)], [float(16 - i) for i in range(32)]],
        expected_matvec=[2464.0, -2464.0])

    # TST/GgufQ8RawTest.java:237-260: 5 blocks against the independent scalar
    # reference (:99-109), vector offset 5, tolerance 1e-3.
    half_scales = [0x3C00, 0x4000, 0xBC00, 0x4200, 0x3800]
    scales = [1.0, 2.0, -1.0, 3.0, 0.5]
    seeds = [11, 29, 47, 83, 109]
    data = []
    for hs, sd in zip(half_scales, seeds):
        data += q8_pattern_block(hs, sd)
    vec = [np.float32((i % 19 - 9) * np.float32(0.0625)) for i in range(5 * 32 + 5)]
    s = np.float32(0.0)
    deq = []
    for b in range(5):
        for i in range(32):
            q = np.int8(np.uint8((seeds[b] + 41 * i) & 0xFF).view(np.int8))
            deq.append(float(np.float32(q) * np.float32(scales[b])))
            s = np.float32(s + np.float32(np.float32(scales[b]) * np.float32(q)) * vec[5 + 32 * b + i])
    add("q8_0_independent_reference", "TST/GgufQ8RawTest.java:237-260", Q8_0, 160, 1, data,
        vector=[float(v) for v in vec], vector_offset=5, expected_dequant=[deq],
        expected_matvec=[float(s)], tolerance=1e-3)

    # fp16 special values (TST/GgufF16SpecialTest.java:18-44) as Q8_0 block
    # scales with every quant = 1, so each block dequantizes to d exactly.
    specials = [0x0000, 0x8000, 0x7C00, 0xFC00, 0x0001, 0x7E00]
    vals = [0.0, -0.0, float("inf"), float("-inf"), 2.0 ** -24, float("nan")]
    data = []
    for h in specials:
        data += q8_block(h, 1)
    nan_bits = struct.unpack("<f", struct.pack("<I", 0x7FC00000))[0]
    add("f16_special_scales", "TST/GgufF16SpecialTest.java:18-44 (RT/GgufQuantTables.java:142-164)",
        Q8_0, 32, 6, data, expected_dequant=[[v if v == v else nan_bits] * 32 for v in vals])
    for has_mins in (False, True):
        row = q5k_lane_row(has_mins)
        dot = float(sum(np.float64(a) * b for a, b in zip(row, ramp(256))))
        assert abs(dot) < 2 ** 24 and dot == int(dot)
        add(f"q5k_lane_order_{'min' if has_mins else 'nomin'}",
            "TST/GgufQ5LaneFx.java:13-24 (TST/GgufQ5CalcFx.java:10-66, TST/GgufQ5Fx.java:13-55)",
            13, 256, 1, q5k_lane_block(has_mins), vector=ramp(256), expected_dequant=[row],
            expected_matvec=[dot])
    q5_off = [0] * 176
    q5_off[0:2] = le16(0x3C00)
    q5_off[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
    q5_off[16:48] = [0xFF] * 32
    q5_off[48:176] = [0x11] * 128
    add("q5k_offset_second_block", "TST/GgufQ5KOffTest.java:19-33 (the tensor's block at offset 176)",
        13, 256, 1, q5_off, vector=ones(256), expected_dequant=[[17.0] * 256],
        expected_matvec=[4352.0])
    row = q6k_lane_row()
    dot = float(sum(np.float64(a) * b for a, b in zip(row, ramp(256))))
    assert abs(dot) < 2 ** 24 and dot == int(dot)
    add("q6k_lane_order", "TST/GgufQ6LaneTest.java:20-41 (TST/GgufQ6LaneFx.java:10-48, TST/GgufQ6Fx.java:26-43)",
        14, 256, 1, q6k_lane_block(), vector=ramp(256), expected_dequant=[row],
        expected_matvec=[dot])
    return fx


def main() -> None:
    OUT.write_text(json.dumps(fixtures(), indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
