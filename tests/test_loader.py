"""AutoAWQ checkpoint loading (tandem_amd/loader.py): a synthetic AutoAWQ checkpoint with separate
q / k / v and gate / up tensors (the oracle's random AWQ recipe) goes into fused W4Linear buffers
on the CPU (column fusion, python/tandem/models/loader.py:41-58), then on the GPU the fused layers
must equal the per-shard oracle products (and SwiGLU of the fused gate_up)."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file
from torch import nn

from oracle import awq_oracle as o
from tandem_amd import loader, model as tmodel
from tandem_amd.layers import linear

H, I, Q, KV = 256, 384, 256, 128  # hidden, intermediate, q and k / v output sizes


class Attn(nn.Module):
    def __init__(self, quant):
        super().__init__()
        self.qkv_proj = linear.make_linear(H, Q + 2 * KV, False, quant)
        self.o_proj = linear.make_linear(Q, H, False, quant)


class Layer(nn.Module):
    def __init__(self, quant):
        super().__init__()
        self.self_attn = Attn(quant)
        self.mlp = tmodel.GatedMLP(H, I, quant)
        self.input_layernorm = nn.LayerNorm(H)


class Model(nn.Module):
    def __init__(self, quant):
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList([Layer(quant)])


def _checkpoint(tmp_path, seed=0):
    """Write model.safetensors with one layer's separate AWQ projections; return the tensors."""
    shapes = {"self_attn.q_proj": (H, Q), "self_attn.k_proj": (H, KV), "self_attn.v_proj": (H, KV),
              "self_attn.o_proj": (Q, H), "mlp.gate_proj": (H, I), "mlp.up_proj": (H, I), "mlp.down_proj": (I, H)}
    tensors, raw = {}, {}
    for i, (name, (k, n)) in enumerate(shapes.items()):
        qw, qz, s, _, _ = o.random_awq(k, n, seed=seed + i)
        raw[name] = (qw, qz, s)
        for suffix, t in (("qweight", qw), ("qzeros", qz), ("scales", s)):
            tensors[f"model.layers.0.{name}.{suffix}"] = torch.from_numpy(np.ascontiguousarray(t))
    tensors["model.layers.0.input_layernorm.weight"] = torch.ones(H)
    tensors["model.layers.0.input_layernorm.bias"] = torch.zeros(H)
    tensors["model.layers.0.self_attn.rotary_emb.inv_freq"] = torch.ones(4)  # ignored
    save_file(tensors, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"quantization_config": {
        "quant_method": "awq", "bits": 4, "group_size": 128, "zero_point": True, "version": "GEMM"}}))
    return raw


def test_quant_config():
    assert loader.QuantConfig.from_dict(None) is None
    q = loader.QuantConfig.from_dict({"quant_method": "awq", "bits": 4, "group_size": 128, "version": "GEMM"})
    assert (q.method, q.bits, q.group_size) == ("awq", 4, 128)
    for bad in ({"quant_method": "gptq", "bits": 4}, {"quant_method": "awq", "bits": 8},
                {"quant_method": "awq", "bits": 4, "version": "gemv"}, {"quant_method": "awq", "bits": 4,
                                                                         "zero_point": False}):
        with pytest.raises(NotImplementedError):
            loader.QuantConfig.from_dict(bad)


def test_fused_sources():
    """A fused model tensor names its checkpoint parts in stacking order, with the output-feature
    axis: dim 1 for the AutoAWQ tensors, dim 0 for dense weights and biases."""
    pre = "model.layers.3.self_attn"
    assert loader.fused_sources(f"{pre}.qkv_proj.qzeros") == ([f"{pre}.{p}_proj.qzeros" for p in "qkv"], 1)
    assert loader.fused_sources(f"{pre}.qkv_proj.bias") == ([f"{pre}.{p}_proj.bias" for p in "qkv"], 0)
    assert loader.fused_sources("model.layers.0.mlp.gate_up_proj.scales") == (
        ["model.layers.0.mlp.gate_proj.scales", "model.layers.0.mlp.up_proj.scales"], 1)
    assert loader.fused_sources("model.layers.0.mlp.gate_up_proj.weight")[1] == 0
    assert loader.fused_sources("model.layers.0.mlp.gate_up_proj.bias") is None
    assert loader.fused_sources("model.layers.0.mlp.experts.3.gate_up_proj.weight") is None
    assert loader.fused_sources("model.layers.0.mlp.down_proj.qweight") is None


def test_plan_prefers_same_named_tensor():
    """A checkpoint that already stores the fused tensor fills it directly; a fused tensor with a
    part absent is reported missing, not half-filled."""
    t = {"a.self_attn.qkv_proj.weight": torch.zeros(6, 2), "model.layers.0.mlp.gate_up_proj.qweight": torch.zeros(1)}
    plans, missing = loader.plan_sources(t, {"a.self_attn.qkv_proj.weight", "a.self_attn.q_proj.weight",
                                             "model.layers.0.mlp.gate_proj.qweight"})
    assert plans == {"a.self_attn.qkv_proj.weight": (["a.self_attn.qkv_proj.weight"], 0)}
    assert missing == ["model.layers.0.mlp.gate_up_proj.qweight"]


def test_load_fuses_awq_columns(tmp_path):
    raw = _checkpoint(tmp_path)
    quant = loader.QuantConfig.from_dict(json.loads((tmp_path / "config.json").read_text())["quantization_config"])
    model = Model(quant)
    loader.load_weights(model, str(tmp_path))
    layer = model.model.layers[0]
    qkv, gate_up = layer.self_attn.qkv_proj, layer.mlp.gate_up_proj
    for j, suffix in enumerate(("qweight", "qzeros", "scales")):
        want = np.concatenate([raw[f"self_attn.{p}_proj"][j] for p in "qkv"], axis=1)
        assert np.array_equal(getattr(qkv, suffix).numpy(), want)
        want = np.concatenate([raw[f"mlp.{p}_proj"][j] for p in ("gate", "up")], axis=1)
        assert np.array_equal(getattr(gate_up, suffix).numpy(), want)
        assert np.array_equal(getattr(layer.mlp.down_proj, suffix).numpy(), raw["mlp.down_proj"][j])
    assert layer.mlp.fused_act and gate_up.silu_mul  # the SwiGLU epilogue is armed before finalize


def test_load_reports_missing_and_mismatched(tmp_path):
    _checkpoint(tmp_path)
    model = Model(loader.QuantConfig("awq", 4, 128))
    model.model.layers[0].extra = nn.Linear(4, 4)
    with pytest.raises(RuntimeError, match="lacks 2 model tensors"):
        loader.load_weights(model, str(tmp_path))
    with pytest.raises(FileNotFoundError):
        loader.load_weights(Model(None), str(tmp_path / "nowhere"))


def test_load_rejects_shape_mismatch_before_copying(tmp_path):
    """A checkpoint whose k_proj is wider than the model's qkv leaves room for raises ValueError, and
    no model tensor has been written."""
    _checkpoint(tmp_path)
    model = Model(loader.QuantConfig("awq", 4, 128))
    model.model.layers[0].self_attn.qkv_proj = linear.make_linear(H, Q + 2 * KV - 8, False, loader.QuantConfig(
        "awq", 4, 128))
    with torch.no_grad():
        for t in loader.model_tensors(model).values():
            t.zero_()  # W4Linear's AutoAWQ buffers start uninitialised
    before = {n: t.clone() for n, t in loader.model_tensors(model).items()}
    with pytest.raises(ValueError, match="qkv_proj"):
        loader.load_weights(model, str(tmp_path))
    assert all(torch.equal(before[n], t) for n, t in loader.model_tensors(model).items())


@pytest.mark.gpu
def test_loaded_layers_on_gpu(tmp_path):
    """Fused qkv = [q | k | v] of the per-shard oracle products; the fused gate_up's SwiGLU output
    equals the oracle's SwiGLU of the separate gate and up, and the MLP feeds it to down_proj
    (the reference's layer tolerances: 0.05 / 0.02, SwiGLU 0.03 / 0.02)."""
    raw = _checkpoint(tmp_path, seed=10)
    model = Model(loader.QuantConfig("awq", 4, 128))
    loader.load_weights(model, str(tmp_path))
    model.to("cuda")
    assert linear.finalize_quantized(model, torch.cuda.get_device_name()) == 4
    layer = model.model.layers[0]
    w = {name: o.dequant_exact(*t) for name, t in raw.items()}
    rng = np.random.default_rng(3)
    for m in (1, 5, 24):
        x = rng.standard_normal((m, H)).astype(np.float16)
        xg = torch.from_numpy(x).cuda()
        y = layer.self_attn.qkv_proj(xg).float().cpu().numpy()
        ref = np.concatenate([o.linear(x, o.dequant(*raw[f"self_attn.{p}_proj"])) for p in "qkv"], axis=1)
        assert np.allclose(y, ref, atol=0.05, rtol=0.02), (m, float(np.abs(y - ref).max()))
        g = layer.mlp.gate_up_proj(xg).float().cpu().numpy()
        ref = o.swiglu_reference(x, np.concatenate([w["mlp.gate_proj"], w["mlp.up_proj"]]))
        assert np.allclose(g, ref, atol=0.03, rtol=0.02), (m, float(np.abs(g - ref).max()))
        d = model.model.layers[0].mlp(xg).float().cpu().numpy()
        ref = o.linear(g.astype(np.float16), o.dequant(*raw["mlp.down_proj"]))
        assert np.allclose(d, ref, atol=0.05, rtol=0.02), (m, float(np.abs(d - ref).max()))
