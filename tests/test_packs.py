"""The checkpoint packer and pack reader (the reference's ``packs/packer.py`` Packer / PackFile and
``formats/checkpoint.py`` grouping): a synthetic checkpoint in the stored conventions (ModelOpt NVFP4 and FP8, MLX
NVFP4 and affine INT4, BF16) is packed into T16 slabs; the reader's float matrix equals the oracle's dequantization of
the same stored tensors (bit for bit, row scales, row subsets, the gate|up interleave and expert stacking included),
and on the GPU the uploaded slab decodes to those bits and feeds the GEMV."""

import numpy as np
import pytest

from helpers import from_dev_bf16, to_dev_bf16
from oracle import formats as OF
from oracle import nn as ON
from oracle.fp import bf16_to_f32, f32_to_bf16, rbf
from oracle.gates import check_against_oracle

K = 256


def _ckpt(tmp_path, rng):
    """Stored tensors of a small model and the oracle dicts they encode."""
    from monolith_mi355.packs import write
    t, ref = {}, {}

    def nvfp4_modelopt(name, n, s2):
        m = OF.nvfp4_random(n, K, rng, s2=s2)
        t[f"{name}.weight"] = (m["weight"], "U8")
        t[f"{name}.weight_scale"] = (m["weight_scale"], "F8_E4M3")
        t[f"{name}.weight_scale_2"] = (np.float32(m["weight_scale_2"]), "F32")
        t[f"{name}.input_scale"] = (np.float32(1.0), "F32")
        ref[name] = m

    nvfp4_modelopt("layers.0.mlp.gate_proj", 64, 0.01)
    nvfp4_modelopt("layers.0.mlp.up_proj", 64, 0.02)
    m = OF.nvfp4_random(48, K, rng, s2=1.0)                                   # MLX nvfp4: U32 codes, U8 scales
    t["layers.0.mlp.down_proj.weight"] = (m["weight"].view(np.uint32), "U32")
    t["layers.0.mlp.down_proj.scales"] = (m["weight_scale"], "U8")
    ref["layers.0.mlp.down_proj"] = m
    m = OF.fp8_random(80, K, rng, s=0.003)
    t["layers.0.attn.q_proj.weight"] = (m["weight"], "F8_E4M3")
    t["layers.0.attn.q_proj.weight_scale"] = (np.float32(m["weight_scale"]), "F32")
    ref["layers.0.attn.q_proj"] = m
    m = OF.int4_random(32, K, rng)
    t["layers.0.attn.o_proj.weight"] = (m["weight"].view(np.uint32), "U32")
    t["layers.0.attn.o_proj.scales"] = (f32_to_bf16(m["scales"]), "BF16")
    t["layers.0.attn.o_proj.biases"] = (f32_to_bf16(m["biases"]), "BF16")
    ref["layers.0.attn.o_proj"] = m
    for e in range(4):
        nvfp4_modelopt(f"layers.0.moe.experts.{e}.gate_proj", 32, 0.01 * (e + 1))
    w = rbf(rng.standard_normal((16, K)) * 0.05)
    t["layers.0.router.weight"] = (f32_to_bf16(w), "BF16")
    ref["layers.0.router"] = {"format": "bf16", "weight": f32_to_bf16(w)}
    t["layers.0.norm.weight"] = (f32_to_bf16(rng.standard_normal(K) * 0.1), "BF16")
    t["layers.0.A_log"] = (rng.standard_normal(8).astype(np.float32), "F32")
    half = {k: v for i, (k, v) in enumerate(t.items()) if i % 2 == 0}            # two shards
    rest = {k: v for k, v in t.items() if k not in half}
    write(tmp_path / "model-1.safetensors", half, {"format": "pt"})
    write(tmp_path / "model-2.safetensors", rest)
    return ref


def _dequant_rows(m):
    return bf16_to_f32(m["weight"]) if m["format"] == "bf16" else OF.dequantize(m)


@pytest.fixture
def packed(tmp_path, rng):
    from monolith_mi355.packs import Packer, PackFile, Segment
    from monolith_mi355.packs.transforms import interleave_chunks
    ck, out = tmp_path / "ckpt", tmp_path / "pack"
    ck.mkdir()
    ref = _ckpt(ck, rng)
    p = Packer(ck, out)
    gu = interleave_chunks(64, 64, 8)
    p.add_slab("gate_up", "nvfp4", [Segment("layers.0.mlp.gate_proj"), Segment("layers.0.mlp.up_proj")], row_perm=gu)
    p.add_slab("down", "nvfp4", [Segment("layers.0.mlp.down_proj")])
    sel = np.array([5, 1, 70, 3] + list(range(10, 22)))
    p.add_slab("q_sel", "fp8_e4m3", [Segment("layers.0.attn.q_proj", rows=sel)])
    p.add_slab("o", "int4_affine", [Segment("layers.0.attn.o_proj")])
    p.add_slab("experts", "nvfp4", [Segment(f"layers.0.moe.experts.{e}.gate_proj") for e in range(4)], experts=4)
    p.add_slab("router", "bf16", [Segment("layers.0.router")])
    p.add_slab("router_q", "nvfp4", [Segment("layers.0.router")])          # a BF16 matrix quantized at pack time
    p.add_aux("norm", "layers.0.norm.weight", transform="one_plus")
    p.add_aux("neg_exp_a", "layers.0.A_log", transform="neg_exp", perm=np.arange(8)[::-1].copy())
    p.add_table("cos", np.arange(12, dtype=np.float32).reshape(3, 4))
    p.write({"model": "synthetic"})
    return PackFile(out), ref, gu, sel


def test_format_detection(tmp_path, rng):
    from monolith_mi355.packs import Checkpoint, group_tensors, logical_shape
    ck = tmp_path / "c"
    ck.mkdir()
    _ckpt(ck, rng)
    c = Checkpoint(ck)
    dt = {n: c.info(n).dtype for n in c.names()}
    g = group_tensors(c.names(), dt)
    assert g["layers.0.mlp.gate_proj"].format == "nvfp4" and "input_scale" in g["layers.0.mlp.gate_proj"].sides
    assert g["layers.0.mlp.down_proj"].format == "nvfp4"
    assert g["layers.0.attn.q_proj"].format == "fp8_e4m3"
    assert g["layers.0.attn.o_proj"].format == "int4_affine"
    assert g["layers.0.router"].format == "bf16"
    shapes = {n: c.info(n).shape for n in c.names()}
    assert logical_shape(g["layers.0.mlp.down_proj"], shapes) == (48, K)          # 8 codes per U32
    assert logical_shape(g["layers.0.mlp.gate_proj"], shapes) == (64, K)          # 2 codes per U8


def test_slabs_dequantize_to_the_stored_matrices(packed):
    pf, ref, gu, sel = packed
    g = OF.dequantize(ref["layers.0.mlp.gate_proj"])
    u = OF.dequantize(ref["layers.0.mlp.up_proj"])
    assert np.array_equal(pf.dequantize_slab("gate_up"), np.concatenate([g, u])[gu])
    assert np.array_equal(pf.dequantize_slab("down"), OF.dequantize(ref["layers.0.mlp.down_proj"]))
    assert np.array_equal(pf.dequantize_slab("q_sel"), OF.dequantize(ref["layers.0.attn.q_proj"])[sel])
    assert np.array_equal(pf.dequantize_slab("o"), OF.dequantize(ref["layers.0.attn.o_proj"]))
    for e in range(4):
        assert np.array_equal(pf.dequantize_slab("experts", e), OF.dequantize(ref[f"layers.0.moe.experts.{e}.gate_proj"]))
    assert np.array_equal(pf.dequantize_slab("router"), _dequant_rows(ref["layers.0.router"]))
    rq = OF.nvfp4_quantize(_dequant_rows(ref["layers.0.router"]))
    assert np.array_equal(pf.dequantize_slab("router_q"), OF.dequantize(rq))
    s = pf.slabs["gate_up"]
    assert [seg["tensor_scale"] for seg in s["segments"]] == [np.float32(0.01), np.float32(0.02)]
    rs = pf.row_scales("gate_up")[:128]
    assert np.array_equal(rs, np.repeat(np.float32([0.01, 0.02]), 64)[gu])
    assert s["offset"] % 4096 == 0 and pf.manifest["model"] == "synthetic"


def test_aux_and_tables(packed, tmp_path):
    pf, ref, gu, sel = packed
    from monolith_mi355.packs import Checkpoint
    c = Checkpoint(tmp_path / "ckpt")
    w = bf16_to_f32(np.asarray(c.get("layers.0.norm.weight")))
    assert np.array_equal(pf.aux_array("norm"), (np.float32(1) + w).astype(np.float32))
    a = np.asarray(c.get("layers.0.A_log"), np.float32)
    assert np.array_equal(pf.aux_array("neg_exp_a"), (-np.exp(bf16_to_f32(f32_to_bf16(a))))[::-1].astype(np.float32))
    assert np.array_equal(pf.aux_array("cos"), np.arange(12, dtype=np.float32).reshape(3, 4))


def test_packer_rejects(tmp_path, rng):
    from monolith_mi355.packs import Packer, Segment
    ck = tmp_path / "c"
    ck.mkdir()
    _ckpt(ck, rng)
    p = Packer(ck, tmp_path / "o")
    with pytest.raises(KeyError):
        p.add_slab("x", "nvfp4", [Segment("nope")])
    with pytest.raises(ValueError):                                  # stored NVFP4 is not re-quantized to FP8
        p.add_slab("x", "fp8_e4m3", [Segment("layers.0.mlp.gate_proj")])
    with pytest.raises(ValueError):
        p.add_slab("x", "nvfp4", [Segment("layers.0.mlp.gate_proj")], row_perm=np.zeros(64, np.int64))
    with pytest.raises(ValueError):                                  # 48 rows are not 2 experts of whole tiles
        p.add_slab("x", "nvfp4", [Segment("layers.0.mlp.down_proj")], experts=2)


@pytest.mark.gpu
def test_uploaded_slabs_decode_and_multiply(torch_gpu, packed, rng):
    from monolith_mi355 import kernels
    pf, ref, gu, sel = packed
    for name in ("gate_up", "down", "q_sel", "o", "router"):
        w = pf.upload(name)
        got = kernels.dequant(w).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), pf.dequantize_slab(name).view(np.uint32)), name
    w = pf.upload("experts")
    for e in range(4):
        got = kernels.dequant(w, expert=e).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), pf.dequantize_slab("experts", e).view(np.uint32)), e
    x = rbf(rng.standard_normal((1, K)))
    got = from_dev_bf16(kernels.gemv(pf.upload("gate_up"), to_dev_bf16(torch_gpu, x), epilogue="silu_mul"))
    wd = np.concatenate([OF.dequantize(ref["layers.0.mlp.gate_proj"]), OF.dequantize(ref["layers.0.mlp.up_proj"])])
    refy = ON.linear(x, wd, epilogue="silu_mul")
    assert check_against_oracle(got, refy).ok_rounded()
