"""The oracle's codecs and quantizers, pinned three ways: the reference's known answers
(``tests/contract/test_fp_codes.py:8-43``, ``tests/contract/test_formats.py:17-44``), brute force over every code,
and golden vectors written by the reference's own ``monolith.formats`` (``tests/golden/formats.npz``). The product's
host and GPU quantizers and the T16 pack are checked against the pinned oracle."""

from pathlib import Path

import numpy as np
import pytest

from oracle import formats as OF
from oracle.fp import (E2M1_TABLE, E4M3_TABLE, bf16_to_f32, e2m1_to_f32, e4m3_to_f32, f32_to_bf16, f32_to_e2m1,
                       f32_to_e4m3, pack_nibbles, unpack_nibbles)

GOLD = np.load(Path(__file__).parent / "golden" / "formats.npz")


# ---- known answers ---------------------------------------------------------------------------------------------
def test_e4m3_known_answers():
    assert E4M3_TABLE[0x00] == 0 and E4M3_TABLE[0x38] == 1.0 and E4M3_TABLE[0x3C] == 1.5
    assert E4M3_TABLE[0x7E] == 448 and np.isnan(E4M3_TABLE[0x7F]) and np.isnan(E4M3_TABLE[0xFF])
    assert E4M3_TABLE[0x08] == 2.0 ** -6 and E4M3_TABLE[0x01] == 2.0 ** -9
    assert np.signbit(E4M3_TABLE[0x80]) and E4M3_TABLE[0xB8] == -1.0
    got = f32_to_e4m3(np.array([1.0625, 1.1875, 500.0, -500.0, np.nan], np.float32)).tolist()
    assert got == [0x38, 0x3A, 0x7E, 0xFE, 0x7F]
    with pytest.raises(ValueError):
        f32_to_e4m3(np.array([1000.0]), saturate=False)


def test_e4m3_brute_force_round_trip_and_rounding():
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    assert np.array_equal(f32_to_e4m3(e4m3_to_f32(codes)), codes)
    # every midpoint between consecutive finite positive values rounds to the even code
    pos = np.arange(0x7F, dtype=np.uint8)
    vals = e4m3_to_f32(pos).astype(np.float64)
    mid = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    exact_mid = mid.astype(np.float64) == (vals[:-1] + vals[1:]) / 2
    want = np.where(pos[:-1] % 2 == 0, pos[:-1], pos[1:])
    assert np.array_equal(f32_to_e4m3(mid)[exact_mid], want[exact_mid])
    # just above / below a midpoint goes to the nearer value
    up = np.nextafter(mid, np.float32(np.inf))
    assert np.array_equal(f32_to_e4m3(up)[exact_mid], pos[1:][exact_mid])


def test_e2m1_known_answers_and_nibbles():
    assert E2M1_TABLE.tolist() == [0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6]
    codes = np.arange(16, dtype=np.uint8)
    assert np.array_equal(f32_to_e2m1(e2m1_to_f32(codes))[1:8], codes[1:8])
    assert f32_to_e2m1(np.array([0.25, 0.75, 2.5, 5.0, 7.0, -0.25], np.float32)).tolist() == [0, 2, 4, 6, 7, 8]
    packed = pack_nibbles(np.array([[1, 2, 3, 4]], np.uint8))
    assert packed.tolist() == [[0x21, 0x43]] and np.array_equal(unpack_nibbles(packed), [[1, 2, 3, 4]])
    with pytest.raises(ValueError):
        e2m1_to_f32(np.array([16], np.uint8))


def test_bf16_known_answers():
    x = np.array([1.0, -2.5, 3.14159, 1e-40, 65504.0], np.float32)
    b = f32_to_bf16(x)
    assert b[0] == 0x3F80 and b[1] == 0xC020
    assert np.allclose(bf16_to_f32(b), x, rtol=2 ** -8)
    assert bf16_to_f32(f32_to_bf16(np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8], np.float32))).tolist() == [1.0, 1 + 2 ** -6]
    assert np.isnan(bf16_to_f32(f32_to_bf16(np.array([np.nan], np.float32))))[0]


# ---- golden vectors from the reference --------------------------------------------------------------------------
def test_codecs_match_reference_golden():
    v = GOLD["codec_in"]
    assert np.array_equal(f32_to_e4m3(v), GOLD["e4m3"])
    assert np.array_equal(f32_to_e2m1(np.clip(v, -6, 6)), GOLD["e2m1"])
    assert np.array_equal(f32_to_bf16(v), GOLD["bf16"])


def test_nvfp4_quantize_dequantize_match_reference_golden():
    q = OF.nvfp4_quantize(GOLD["nv_w"])
    assert np.array_equal(q["weight"], GOLD["nv_codes"]) and np.array_equal(q["weight_scale"], GOLD["nv_scales"])
    assert np.float32(q["weight_scale_2"]) == GOLD["nv_s2"]
    assert np.array_equal(OF.nvfp4_dequantize(q).view(np.uint32), GOLD["nv_deq"].view(np.uint32))


def test_int4_quantize_dequantize_match_reference_golden():
    q = OF.int4_quantize(GOLD["i4_w"])
    assert np.array_equal(q["weight"], GOLD["i4_codes"])
    assert np.array_equal(q["scales"], GOLD["i4_scales"]) and np.array_equal(q["biases"], GOLD["i4_biases"])
    assert np.array_equal(OF.int4_dequantize(q).view(np.uint32), GOLD["i4_deq"].view(np.uint32))


def test_nvfp4_dequant_per_element_formula():
    """The reference's per-element formula test (tests/contract/test_formats.py:33-44)."""
    rng = np.random.default_rng(0)
    q = OF.nvfp4_quantize((rng.standard_normal((8, 64)) * 0.02).astype(np.float32))
    codes = unpack_nibbles(q["weight"])
    ref = np.empty((8, 64), np.float32)
    for n in range(8):
        for k in range(64):
            ref[n, k] = e2m1_to_f32(codes[n, k]) * e4m3_to_f32(q["weight_scale"][n, k // 16]) * np.float32(q["weight_scale_2"])
    assert np.array_equal(OF.nvfp4_dequantize(q), ref)


def test_quantizers_error_bounds_and_requantize():
    """quantize→dequantize error bounds and idempotence (tests/contract/test_formats.py:17-30)."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((40, 1024)) * 0.02).astype(np.float32)
    for fmt, tol in (("nvfp4", 0.35), ("int4_affine", 0.12)):
        wq = OF.dequantize(OF.quantize(fmt, w))
        assert np.sqrt(np.mean((wq - w) ** 2)) / np.sqrt(np.mean(w ** 2)) < tol
        wqq = OF.dequantize(OF.quantize(fmt, wq))
        if fmt == "nvfp4":
            assert np.array_equal(wqq, wq)
        else:
            step = np.repeat(np.abs(OF.quantize(fmt, wq)["scales"]), 64, axis=1)
            assert np.all(np.abs(wqq - wq) <= step + 1e-7) and np.mean(wqq == wq) > 0.7


def test_int4_dequant_closed_form_single_rounding():
    """code·scale is exact (BF16 scale × 4-bit code), so numpy's two roundings equal one fused rounding."""
    rng = np.random.default_rng(2)
    m = OF.int4_random(16, 256, rng)
    codes = unpack_nibbles(m["weight"]).astype(np.float64)
    sc = np.repeat(m["scales"].astype(np.float64), 64, axis=1)
    bi = np.repeat(m["biases"].astype(np.float64), 64, axis=1)
    assert np.array_equal(OF.int4_dequantize(m), (codes * sc + bi).astype(np.float32))


# ---- the product's quantizers and pack against the pinned oracle ---------------------------------------------------
def test_product_quantizers_match_oracle():
    from monolith_mi355.formats import FORMATS
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((48, 512)) * 0.02).astype(np.float32)
    w[2, :16] = 0.0
    a, b = FORMATS["nvfp4"].quantize(w), OF.nvfp4_quantize(w)
    assert np.array_equal(a.tensors["weight"], b["weight"]) and np.array_equal(a.tensors["weight_scale"], b["weight_scale"])
    assert a.params["weight_scale_2"] == b["weight_scale_2"]
    a, b = FORMATS["int4_affine"].quantize(w), OF.int4_quantize(w)
    assert np.array_equal(a.tensors["weight"], b["weight"]) and np.array_equal(a.tensors["scales"], b["scales"])
    assert np.array_equal(a.tensors["biases"], b["biases"])


def test_product_e4m3_encoder_every_midpoint():
    from monolith_mi355.formats import e4m3_decode, e4m3_encode
    v = np.concatenate([GOLD["codec_in"], np.linspace(-500, 500, 20001, dtype=np.float32),
                        (np.arange(1, 300, dtype=np.float32) * 2.0 ** -12)]).astype(np.float32)
    assert np.array_equal(e4m3_encode(v), f32_to_e4m3(v))
    codes = np.arange(256, dtype=np.uint8)
    assert np.array_equal(e4m3_decode(codes), E4M3_TABLE, equal_nan=True)


def test_device_quantizer_and_pack_match_host():
    torch = pytest.importorskip("torch")
    from monolith_mi355.formats import FORMATS
    from monolith_mi355.formats import device as DV
    from monolith_mi355.formats import pack as P
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((40, 512)) * 0.02).astype(np.float32)
    w[1, 16:32] = 0.0
    spec = FORMATS["nvfp4"].quantize(w)
    c, sc, s2 = DV.nvfp4_quantize(torch.from_numpy(w))
    assert np.array_equal(c.numpy(), spec.tensors["weight"]) and np.array_equal(sc.numpy(), spec.tensors["weight_scale"])
    assert s2 == spec.params["weight_scale_2"]
    data, _ = P.pack(spec)
    assert np.array_equal(DV.pack_nvfp4(c, sc).numpy(), data)


@pytest.mark.parametrize("fmt", ["nvfp4", "int4_affine", "bf16"])
@pytest.mark.parametrize("n,k", [(37, 512), (16, 128), (100, 1024), (20, 1664), (33, 2304)])
def test_t16_pack_round_trip_and_unit_map(fmt, n, k):
    from monolith_mi355.formats import FORMATS
    from monolith_mi355.formats import pack as P
    if fmt == "bf16" and k % 32:
        pytest.skip()
    rng = np.random.default_rng(n * k)
    spec = FORMATS[fmt].quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    data, info = P.pack(spec)
    assert data.size == P.pack_bytes(fmt, n, k) == info.nbytes
    back = P.unpack(data, info)
    assert np.array_equal(FORMATS[fmt].dequantize(back), FORMATS[fmt].dequantize(spec))
    # lane 21 of tile 1, chunk 0: row 16 + 5, k-group 1 (codes in the chunk's block, scales in the group's piece)
    if fmt == "nvfp4" and n > 21:
        groups, tile_b = P.nvfp4_groups(info.chunks)
        tile = data[tile_b:][:tile_b]
        g0 = groups[0][1]
        piece = 16 if g0 > 4 else 8
        assert np.array_equal(tile[16 * 21: 16 * 22], spec.tensors["weight"][21, 16:32])
        assert np.array_equal(tile[g0 * 1024 + piece * 21: g0 * 1024 + piece * 21 + 2], spec.tensors["weight_scale"][21, 2:4])
        if info.chunks > 1:      # chunk 1 of the group: the next two bytes of the same piece
            assert np.array_equal(tile[g0 * 1024 + piece * 21 + 2: g0 * 1024 + piece * 21 + 4],
                                  spec.tensors["weight_scale"][21, 10:12])


# ---- FP8 E4M3 (formats/fp8_e4m3.py) --------------------------------------------------------------------------------
def test_fp8_dequantize_is_code_times_scale():
    """``w = e4m3(code) · s`` with one rounding; e4m3 itself is pinned by the code-table tests above."""
    from oracle.fp import e4m3_to_f32
    codes = np.arange(256, dtype=np.uint8).reshape(4, 64)
    s = 0.0123
    got = OF.fp8_dequantize({"format": "fp8_e4m3", "weight": codes, "weight_scale": s})
    fin = (codes & 0x7F) != 0x7F
    ref = e4m3_to_f32(codes).astype(np.float64) * np.float64(np.float32(s))
    assert np.array_equal(got[fin], ref[fin].astype(np.float32))          # one rounding of the exact product
    assert np.signbit(got[0, 0]) == False and np.signbit(got[2, 0]) == True and got[2, 0] == 0.0   # ±0


def test_fp8_quantize_closed_form(rng):
    """s = amax / 448 exactly; the largest |w| maps to ±448 (code 0x7E / 0xFE); every code is the nearest E4M3 of
    w / s (within half an E4M3 step); quantize∘dequantize is idempotent on the codes."""
    from oracle.fp import e4m3_to_f32
    w = (rng.standard_normal((64, 128)) * 0.05).astype(np.float32)
    m = OF.fp8_quantize(w)
    amax = float(np.abs(w).max())
    assert m["weight_scale"] == float(np.float32(amax / 448.0))
    i = np.unravel_index(np.argmax(np.abs(w)), w.shape)
    assert m["weight"][i] in (0x7E, 0xFE)
    v = e4m3_to_f32(m["weight"])
    x = w / np.float32(m["weight_scale"])
    step = np.maximum(2.0 ** (np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -6))) - 3), 2.0 ** -9)
    assert np.all(np.abs(v - x) <= step / 2 + 1e-12)
    again = OF.fp8_quantize(OF.fp8_dequantize(m))
    assert np.array_equal(again["weight"], m["weight"])


def test_fp8_host_format_matches_oracle(rng):
    from monolith_mi355.formats import FORMATS
    w = (rng.standard_normal((32, 256)) * 0.03).astype(np.float32)
    spec = FORMATS["fp8_e4m3"].quantize(w)
    m = OF.fp8_quantize(w)
    assert np.array_equal(spec.tensors["weight"], m["weight"]) and spec.params["weight_scale"] == m["weight_scale"]
    assert np.array_equal(FORMATS["fp8_e4m3"].dequantize(spec), OF.fp8_dequantize(m))


@pytest.mark.parametrize("n,k", [(16, 64), (37, 512), (300, 1024)])
def test_fp8_pack_round_trip(n, k, rng):
    """The T16 FP8 pack: lane l of chunk c holds row l % 16, columns 64c + 16(l // 16) + [0, 16); unpack inverts it."""
    from monolith_mi355.formats import pack as P
    from monolith_mi355.formats import DequantSpec
    m = OF.fp8_random(n, k, rng)
    data, info = P.pack(DequantSpec("fp8_e4m3", (n, k), {"weight": m["weight"]}, {"weight_scale": m["weight_scale"]}))
    assert data.size == P.pack_bytes("fp8_e4m3", n, k) == -(-n // 16) * (k // 64) * 1024
    back = P.unpack(data, info)
    assert np.array_equal(back.tensors["weight"], m["weight"]) and back.params["weight_scale"] == m["weight_scale"]
    t, c, lane = (n - 1) // 16, (k // 64) - 1, 37
    r, g = lane % 16, lane // 16
    unit = data.reshape(-1, k // 64, 1024)[t, c]
    row = t * 16 + r
    if row < n:
        assert np.array_equal(unit[16 * lane: 16 * lane + 16], m["weight"][row, 64 * c + 16 * g: 64 * c + 16 * g + 16])
