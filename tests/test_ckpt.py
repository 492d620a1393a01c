"""Quantized-checkpoint loader (include/mi_ckpt.h) against handmade MLX checkpoints.

Files are written with the safetensors package (an independent writer of the
format), so a header or offset mistake in the loader's reader shows as a byte
mismatch. Expected parameters follow the reference's own config tests
(src/model.zig:3196, 3860, 3926, 4064, 4365) and computeQuantParams
(src/transformer.zig:16876-16924); the f16->bf16 narrowing is checked against
torch's own conversion.
"""
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle as O
from helpers import BF16_TOL, max_err_ratio, to_dev_bf16, to_f64
import mi_qmm
from mi_qmm import Checkpoint, MiError, parse_quant_config


def _u32(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).view(torch.uint32)


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def _affine_layer(prefix, N, K, bits, gs, seed):
    w = O.f32_to_bf16(O.randn(N * K, seed, 0.0, 0.02).reshape(N, K))
    wq, s, b = O.quantize(w, gs, bits)
    return {prefix + ".weight": _u32(wq), prefix + ".scales": _bf16(s),
            prefix + ".biases": _bf16(b)}, (wq, s, b)


def _model_dir(tmp_path, quant, shards):
    if quant is not None:
        (tmp_path / "config.json").write_text(json.dumps(
            {"model_type": "llama", "hidden_size": 64, "quantization": quant}))
    for i, tensors in enumerate(shards):
        save_file(tensors, str(tmp_path / f"model-{i:05d}-of-{len(shards):05d}.safetensors"),
                  metadata={"format": "mlx"})
    return tmp_path


# ---------------------------------------------------------------- config block ---

@pytest.mark.parametrize("quant,expect", [
    (None, (0, 64, "affine")),                                         # model.zig:3196
    ({"bits": 4, "group_size": 64}, (4, 64, "affine")),                # model.zig:3860
    ({"group_size": 16, "bits": 4, "mode": "nvfp4"}, (4, 16, "nvfp4")),  # model.zig:3926
    ({"group_size": 64, "bits": 8}, (8, 64, "affine")),                # model.zig:4064
    ({"group_size": 32, "bits": 4, "mode": "mxfp4"}, (4, 32, "mxfp4")),
    ({"group_size": 32, "bits": 8, "mode": "mxfp8"}, (8, 32, "mxfp8")),
    ({"group_size": 64, "bits": 4, "recipe": "uniform"}, (4, 64, "affine")),  # model.zig:4251
    ({"group_size": 64, "bits": 8, "mode": "affine",                   # model.zig:4365
      "layers.0.ffn.experts.w1": {"group_size": 64, "bits": 2, "mode": "affine"}},
     (8, 64, "affine")),
    ({"bits": 3}, (3, 64, "affine")),                                  # default gs kept
])
def test_parse_quant_config(quant, expect):
    cfg = {"model_type": "x", "text_config": {"hidden_size": 8}}
    if quant is not None:
        cfg["quantization"] = quant
    assert parse_quant_config(json.dumps(cfg, indent=2)) == expect


@pytest.mark.parametrize("quant,needle", [
    ({"bits": 4, "group_size": 64, "mode": "int4"}, "unsupported quantization mode 'int4'"),
    ({"bits": 7, "group_size": 64}, "7-bit"),
    ({"bits": 1, "group_size": 64}, "1-bit"),
    ({"bits": 4, "group_size": 0}, "group_size"),
])
def test_parse_quant_config_rejects(quant, needle):
    with pytest.raises(MiError, match=needle):
        parse_quant_config(json.dumps({"quantization": quant}))


def test_parse_quant_config_json_edges():
    # Escapes, unicode and nesting must not confuse the reader.
    text = ('{"name": "a\\"b\\u00e9\\ud83d\\ude00", "arr": [1, -2.5e3, true, null, {"x": []}],'
            ' "quantization": {"bits": 5, "group_size": 128}}')
    assert parse_quant_config(text) == (5, 128, "affine")
    for bad in ('{"quantization": {"bits": 4,}', '{"quantization": 4}', '[1, 2]',
                '{"a": "unterminated}', '{"a": 1} trailing', '{"a": "\\ud800"}',
                b'{"a": "\xff"}'):
        with pytest.raises(MiError):
            parse_quant_config(bad)


# ------------------------------------------------------------- tensors + binding ---

def test_affine_dir_roundtrip_and_binding(tmp_path):
    t0, (wq0, s0, b0) = _affine_layer("model.layers.0.mlp.gate_proj", 96, 256, 4, 64, 11)
    t1, (wq1, s1, b1) = _affine_layer("model.layers.0.mlp.down_proj", 64, 384, 4, 64, 12)
    t1["model.norm.weight"] = torch.ones(64, dtype=torch.bfloat16)
    d = _model_dir(tmp_path, {"bits": 4, "group_size": 64}, [t0, t1])
    with Checkpoint(d) as ck:
        assert ck.quant_config == (4, 64, "affine")
        assert ck.names() == sorted(list(t0) + list(t1))
        for name, ref in list(t0.items()) + list(t1.items()):
            got = ck.read(name)
            assert got.dtype == ref.dtype and tuple(got.shape) == tuple(ref.shape)
            assert torch.equal(got.view(torch.uint8), ref.contiguous().view(torch.uint8)), name
        lin = ck.linear("model.layers.0.mlp.gate_proj")
        assert lin == dict(bits=4, group_size=64, mode="affine", has_scales=True,
                           has_biases=True, out_dim=96, in_dim=256)
        w, s, b, p = ck.load_linear("model.layers.0.mlp.down_proj", in_dim=384)
        assert p["in_dim"] == 384 and p["out_dim"] == 64
        # What was loaded dequantizes to exactly what was written.
        got = O.dequantize(w.view(torch.int32).numpy().view(np.uint32),
                           s.view(torch.int16).numpy().view(np.uint16),
                           b.view(torch.int16).numpy().view(np.uint16), 64, 4)
        np.testing.assert_array_equal(got, O.dequantize(wq1, s1, b1, 64, 4))
        with pytest.raises(MiError, match="MISSING WEIGHT: model.layers.0.mlp.up_proj.weight"):
            ck.linear("model.layers.0.mlp.up_proj")
        assert "model.norm.weight" in ck and "nope" not in ck


def test_mixed_precision_geometry(tmp_path):
    # An 8-bit tensor and a 5-bit/gs-128 sidecar inside a 4-bit/gs-64 trunk.
    t, _ = _affine_layer("a", 32, 256, 4, 64, 1)
    t8, _ = _affine_layer("b", 32, 256, 8, 64, 2)
    t5, _ = _affine_layer("c", 32, 512, 5, 128, 3)
    d = _model_dir(tmp_path, {"bits": 4, "group_size": 64}, [{**t, **t8, **t5}])
    with Checkpoint(d) as ck:
        assert ck.linear("a", 256)["bits"] == 4
        # affineParamsFromGeometry with the hint, detectQuantBits without it.
        assert (ck.linear("b", 256)["bits"], ck.linear("b")["bits"]) == (8, 8)
        p = ck.linear("c", 512)
        assert (p["bits"], p["group_size"], p["in_dim"]) == (5, 128, 512)
        # Without the hint the declared gs is assumed: bits = w_cols*32/(s_cols*64).
        assert ck.linear("c")["group_size"] == 64


def _fp_layer(prefix, N, K, mode, seed, with_bias=False):
    bits, gs = {"nvfp4": (4, 16), "mxfp4": (4, 32), "mxfp8": (8, 32)}[mode]
    g = torch.Generator().manual_seed(seed)
    wq = torch.randint(0, 2**31 - 1, (N, K * bits // 32), generator=g).to(torch.uint32)
    sc = torch.randint(100, 140, (N, K // gs), generator=g).to(torch.uint8)
    t = {prefix + ".weight": wq, prefix + ".scales": sc}
    if with_bias:
        t[prefix + ".biases"] = torch.zeros(N, K // gs, dtype=torch.bfloat16)
    return t


def test_fp_modes_and_overrides(tmp_path):
    t = _fp_layer("experts", 64, 256, "nvfp4", 1)
    t.update(_fp_layer("embed", 64, 256, "mxfp8", 2))
    shared, _ = _affine_layer("shared", 64, 256, 8, 64, 3)  # affine override, has biases
    t.update(shared)
    d = _model_dir(tmp_path, {"group_size": 16, "bits": 4, "mode": "nvfp4"}, [t])
    with Checkpoint(d) as ck:
        p = ck.linear("experts", 256)
        assert (p["bits"], p["group_size"], p["mode"], p["has_biases"]) == (4, 16, "nvfp4", False)
        # A per-tensor format inside the fp family is solved from geometry.
        p = ck.linear("embed", 256)
        assert (p["bits"], p["group_size"], p["mode"]) == (8, 32, "mxfp8")
        # Without the hint the model-wide declaration holds.
        assert ck.linear("embed")["mode"] == "nvfp4"
        p = ck.linear("shared", 256)
        assert (p["bits"], p["group_size"], p["mode"], p["has_biases"]) == (8, 64, "affine", True)
        # Unhinted affine override: mlx-lm's default gs 64, bits from bits*gs.
        p = ck.linear("shared")
        assert (p["bits"], p["group_size"]) == (8, 64)


def test_mxfp8_tensor_in_affine_model(tmp_path):
    t = _fp_layer("x", 32, 256, "mxfp8", 5)
    t["x.biases"] = torch.zeros(32, 8, dtype=torch.bfloat16)
    d = _model_dir(tmp_path, {"bits": 4, "group_size": 64}, [t])
    with Checkpoint(d) as ck:
        p = ck.linear("x")
        assert (p["bits"], p["group_size"], p["mode"]) == (8, 32, "mxfp8")


def test_dense_checkpoint(tmp_path):
    d = _model_dir(tmp_path, None, [{"l.weight": torch.zeros(8, 16, dtype=torch.bfloat16)}])
    with Checkpoint(d) as ck:
        assert ck.quant_config == (0, 64, "affine")
        p = ck.linear("l")
        assert not p["has_scales"] and not p["has_biases"] and p["in_dim"] == 16


def test_missing_side_tensors(tmp_path):
    t, _ = _affine_layer("l", 32, 128, 4, 64, 7)
    del t["l.biases"]
    d = _model_dir(tmp_path, {"bits": 4, "group_size": 64}, [t])
    with Checkpoint(d) as ck:
        with pytest.raises(MiError, match="MISSING WEIGHT: l.biases"):
            ck.linear("l")
    del t["l.scales"]
    os.remove(next(str(p) for p in tmp_path.glob("*.safetensors")))
    _model_dir(tmp_path, {"bits": 4, "group_size": 64}, [t])
    with Checkpoint(tmp_path) as ck:
        with pytest.raises(MiError, match="MISSING WEIGHT: l.scales"):
            ck.linear("l")


def test_f16_narrowing(tmp_path, monkeypatch):
    g = torch.Generator().manual_seed(3)
    vals = torch.randn(4, 64, generator=g) * 1e-3
    special = torch.tensor([0.0, -0.0, 6.1e-5, 5.96e-8, -3.0e-6, 65504.0, float("inf"),
                            float("nan"), 1.0 + 2 ** -10, 1.0 + 3 * 2 ** -10], dtype=torch.float32)
    sc = torch.cat([vals.flatten(), special]).to(torch.float16)[:256].reshape(4, 64)
    sc.view(-1)[:special.numel()] = special.to(torch.float16)
    t = {"l.weight": torch.zeros(4, 8, dtype=torch.uint32), "l.scales": sc,
         "l.biases": sc.flip(1).contiguous(), "norm.weight": sc[0].clone(),
         "mat": sc.clone()}
    d = _model_dir(tmp_path, {"bits": 4, "group_size": 64}, [t])
    with Checkpoint(d) as ck:
        for n in ("l.scales", "l.biases", "norm.weight"):
            got = ck.read(n)
            assert got.dtype == torch.bfloat16, n
            want = t[n].to(torch.bfloat16)
            assert torch.equal(got.view(torch.int16)[~want.isnan()],
                               want.view(torch.int16)[~want.isnan()]), n
            assert torch.equal(got.isnan(), want.isnan())
        assert ck.read("mat").dtype == torch.float16  # matmul operands keep their dtype
    monkeypatch.setenv("MLX_SERVE_F16_NARROW_1D", "0")
    with Checkpoint(d) as ck:
        assert ck.read("norm.weight").dtype == torch.float16
        assert ck.read("l.scales").dtype == torch.bfloat16  # side-tensor arm is not switchable


def test_vision_keys_and_later_file_wins(tmp_path):
    shards = [{"vision_tower.p": torch.zeros(2), "audio_tower.p": torch.zeros(2),
               "model.visual.p": torch.zeros(2), "x": torch.zeros(3)},
              {"x": torch.ones(3), "model.encoder.vision_tower.q": torch.zeros(1)}]
    d = _model_dir(tmp_path, None, shards)
    with Checkpoint(d) as ck:
        assert ck.names() == ["x"]
        assert torch.equal(ck.read("x"), torch.ones(3))
    with Checkpoint(d, load_vision=True) as ck:
        assert ck.names() == ["model.visual.p", "vision_tower.p", "x"]


def test_single_file_and_set_quant(tmp_path):
    t, _ = _affine_layer("mtp.fc", 32, 256, 5, 128, 9)
    save_file(t, str(tmp_path / "mtp.safetensors"))
    with Checkpoint(tmp_path / "mtp.safetensors", single_file=True) as ck:
        assert ck.quant_config[0] == 0
        ck.set_quant_config(4, 64)
        p = ck.linear("mtp.fc", 256)
        assert (p["bits"], p["group_size"]) == (5, 128)


def test_bad_files(tmp_path):
    with pytest.raises(MiError, match="no usable weights"):
        Checkpoint(tmp_path)
    (tmp_path / "config.json").write_text('{"quantization": {"bits": 4}}')
    with pytest.raises(MiError, match="incomplete checkpoint"):
        Checkpoint(tmp_path)
    good = tmp_path / "a.safetensors"
    save_file({"x": torch.arange(8, dtype=torch.int32)}, str(good))
    raw = good.read_bytes()
    bad = tmp_path / "b.safetensors"
    bad.write_bytes(raw[:-4])  # truncated data
    with pytest.raises(MiError, match="data_offsets out of range"):
        Checkpoint(tmp_path)
    hlen = int.from_bytes(raw[:8], "little")
    hdr = json.loads(raw[8:8 + hlen])
    hdr["x"]["shape"] = [9]
    h2 = json.dumps(hdr).encode()
    bad.write_bytes(len(h2).to_bytes(8, "little") + h2 + raw[8 + hlen:])
    with pytest.raises(MiError, match="does not match its shape"):
        Checkpoint(tmp_path)
    bad.write_bytes((1 << 40).to_bytes(8, "little") + b"{}")
    with pytest.raises(MiError, match="header length"):
        Checkpoint(tmp_path)
    bad.write_bytes(b"\x03\x00")
    with pytest.raises(MiError, match="too short"):
        Checkpoint(tmp_path)


# --------------------------------------------------------------- into the matmul ---

@pytest.mark.gpu
def test_loaded_layer_matmul(dev, tmp_path):
    N, K, gs, bits = 512, 1024, 64, 4
    t, (wq, s, b) = _affine_layer("model.layers.3.self_attn.o_proj", N, K, bits, gs, 21)
    d = _model_dir(tmp_path, {"bits": bits, "group_size": gs}, [t])
    x = O.make_x_bf16(4, K, 22)
    with Checkpoint(d) as ck:
        w_d, s_d, b_d, p = ck.load_linear("model.layers.3.self_attn.o_proj", K, device=dev)
    assert w_d.is_cuda and (p["bits"], p["group_size"]) == (bits, gs)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), w_d.view(torch.int32), s_d, b_d, True,
                                p["group_size"], p["bits"])
    truth = O.qmm_f64(x, wq, s, b, gs, bits)
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL
