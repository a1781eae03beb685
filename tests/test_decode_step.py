"""The decode step around the projections: the norm kernels (tw4_rms_norm / tw4_add_rms_norm)
against the oracle, a small W4A16 decoder (tandem_amd.model) against a numpy restatement of the
same step built from the oracle's pieces, and the bucketed HIP-graph runner (tandem_amd.decode_graph)
against eager runs of the same model (python/tandem/executor/cuda_graph.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import awq_oracle as o
from tandem_amd import decode_graph, model as tmodel
from tandem_amd.loader import QuantConfig

TINY = tmodel.DecoderConfig(hidden_size=512, intermediate_size=1024, num_heads=4, num_kv_heads=2, head_dim=128,
                            num_layers=2, vocab_size=1000, rms_norm_eps=1e-6)
AWQ = QuantConfig("awq", 4, 128)


# ------------------------------------------------------------------------------------- CPU
def test_bucket_sizes():
    """python/tandem/executor/cuda_graph.py:34-38."""
    assert decode_graph.bucket_sizes(1) == [1]
    assert decode_graph.bucket_sizes(3) == [1, 2, 3]
    assert decode_graph.bucket_sizes(8) == [1, 2, 4, 8]
    assert decode_graph.bucket_sizes(20) == [1, 2, 4, 8, 16, 20]
    assert decode_graph.bucket_sizes(32) == [1, 2, 4, 8, 16, 24, 32]
    with pytest.raises(ValueError):
        decode_graph.bucket_sizes(0)


def test_config_from_hf():
    hf = {"hidden_size": 4096, "intermediate_size": 12288, "num_attention_heads": 32, "num_key_value_heads": 8,
          "head_dim": 128, "num_hidden_layers": 36, "vocab_size": 151936, "rms_norm_eps": 1e-6,
          "tie_word_embeddings": False}
    assert tmodel.DecoderConfig.from_hf(hf) == tmodel.QWEN3_8B


def test_model_parameter_names():
    """Checkpoint names (python/tandem/models/llama_family.py:1-8) with the fused projections."""
    with torch.device("meta"):
        m = tmodel.DecoderModel(TINY, AWQ)
    names = {n for n, _ in m.named_parameters()} | {n for n, _ in m.named_buffers()}
    for want in ("model.embed_tokens.weight", "model.norm.weight", "lm_head.weight",
                 "model.layers.1.self_attn.qkv_proj.qweight", "model.layers.1.self_attn.o_proj.scales",
                 "model.layers.0.mlp.gate_up_proj.qzeros", "model.layers.0.mlp.down_proj.qweight",
                 "model.layers.0.input_layernorm.weight", "model.layers.0.post_attention_layernorm.weight"):
        assert want in names, want
    assert all(layer.mlp.fused_act for layer in m.model.layers)


def test_attend_one_token_is_grouped_value_broadcast():
    """Softmax over one key is 1: head h's output is the value of KV head h // group."""
    attn = tmodel.Attention(TINY, None)
    qkv = torch.randn(3, attn.q_size + 2 * attn.kv_size)
    out = attn.attend(qkv).view(3, TINY.num_heads, TINY.head_dim)
    v = qkv[:, attn.q_size + attn.kv_size:].view(3, TINY.num_kv_heads, TINY.head_dim)
    group = TINY.num_heads // TINY.num_kv_heads
    for h in range(TINY.num_heads):
        assert torch.equal(out[:, h], v[:, h // group])
    q = qkv[:, :attn.q_size].view(3, TINY.num_heads, TINY.head_dim)
    k = qkv[:, attn.q_size:attn.q_size + attn.kv_size].view(3, TINY.num_kv_heads, TINY.head_dim)
    for h in range(TINY.num_heads):  # the same through softmax(q k^T / sqrt(d)) v over one key
        scores = (q[:, h] * k[:, h // group]).sum(-1, keepdim=True) / TINY.head_dim ** 0.5
        assert torch.allclose(torch.softmax(scores, -1) * v[:, h // group], out[:, h])


# ------------------------------------------------------------------------------- GPU helpers
def _tiny_model(seed: int = 0):
    """The tiny decoder with oracle-generated AWQ tensors and seeded fp16 parameters; returns the
    model on the GPU (prepared) and the numpy weights of the step."""
    rng = np.random.default_rng(seed)
    m = tmodel.DecoderModel(TINY, AWQ)
    w = {"layers": []}
    i = 0
    for layer in m.model.layers:
        lw = {}
        for name, lin in (("qkv", layer.self_attn.qkv_proj), ("o", layer.self_attn.o_proj),
                          ("gate_up", layer.mlp.gate_up_proj), ("down", layer.mlp.down_proj)):
            qw, qz, s, _, _ = o.random_awq(lin.in_features, lin.out_features, seed=seed * 100 + i)
            i += 1
            lin.qweight.copy_(torch.from_numpy(qw))
            lin.qzeros.copy_(torch.from_numpy(qz))
            lin.scales.copy_(torch.from_numpy(s))
            lw[name] = o.dequant(qw, qz, s)  # fp16 [N, K], the weights the kernels multiply by
        for name, mod in (("n1", layer.input_layernorm), ("n2", layer.post_attention_layernorm)):
            v = (1.0 + (rng.random(TINY.hidden_size) - 0.5) * 0.2).astype(np.float16)
            mod.weight.data = torch.from_numpy(v.astype(np.float32))
            lw[name] = v
        w["layers"].append(lw)
    emb = rng.standard_normal((TINY.vocab_size, TINY.hidden_size)).astype(np.float16)
    head = (rng.standard_normal((TINY.vocab_size, TINY.hidden_size)) * 0.02).astype(np.float16)
    fn = (1.0 + (rng.random(TINY.hidden_size) - 0.5) * 0.2).astype(np.float16)
    m.model.embed_tokens.weight.data = torch.from_numpy(emb.astype(np.float32))
    m.lm_head.weight.data = torch.from_numpy(head.astype(np.float32))
    m.model.norm.weight.data = torch.from_numpy(fn.astype(np.float32))
    w.update(emb=emb, head=head, norm=fn)
    dev = torch.device("cuda", 0)
    tmodel.prepare(m, dev, torch.cuda.get_device_name(dev))
    return m, w


def _oracle_step(w, ids) -> np.ndarray:
    """The decode step restated with the oracle's norms and float64 products, rounded to fp16
    where the GPU path stores fp16 (python/tandem/models/llama_family.py:47-67, 90-116)."""
    eps = TINY.rms_norm_eps
    hidden = w["emb"][ids]
    residual = None
    q_size, kv = TINY.num_heads * TINY.head_dim, TINY.num_kv_heads * TINY.head_dim
    group = TINY.num_heads // TINY.num_kv_heads
    for lw in w["layers"]:
        if residual is None:
            residual = hidden
            hidden = o.rms_norm(hidden, lw["n1"], eps)
        else:
            hidden, residual = o.add_rms_norm(hidden, residual, lw["n1"], eps)
        qkv = o.linear(hidden, lw["qkv"]).astype(np.float16)
        v = qkv[:, q_size + kv:].reshape(len(ids), TINY.num_kv_heads, 1, TINY.head_dim)
        attn = np.broadcast_to(v, (len(ids), TINY.num_kv_heads, group, TINY.head_dim)).reshape(len(ids), q_size)
        hidden = o.linear(attn, lw["o"]).astype(np.float16)
        hidden, residual = o.add_rms_norm(hidden, residual, lw["n2"], eps)
        gu = o.linear(hidden, lw["gate_up"])
        hidden = o.silu_and_mul(gu).astype(np.float16)
        hidden = o.linear(hidden, lw["down"]).astype(np.float16)
    hidden, _ = o.add_rms_norm(hidden, residual, w["norm"], eps)
    return o.linear(hidden, w["head"])


def _close(y: torch.Tensor, ref: np.ndarray, rtol: float, what) -> None:
    got = y.detach().float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-6)
    cos = (got * ref).sum() / np.sqrt((got * got).sum() * (ref * ref).sum())
    assert err <= rtol and cos >= 0.9999, (what, err, cos)


# ----------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("k", [512, 1024, 2048, 2560, 3584, 4096, 5120, 8192])
def test_norm_kernels_match_oracle(k):
    """Residual bit-exact; normalised output within one fp16 ulp of the oracle's float64 result
    (the kernel's fp32 sum and two fp32 products round differently near ties)."""
    from tandem_amd.layers import norm

    rng = np.random.default_rng(k)
    for m in (1, 3, 4, 5, 9):
        x = (rng.standard_normal((m, k)) * 3).astype(np.float16)
        r = (rng.standard_normal((m, k)) * 20).astype(np.float16)
        w = (rng.random(k) + 0.5).astype(np.float16)
        eps = 1e-6
        xg, rg, wg = (torch.from_numpy(a).cuda() for a in (x, r, w))
        y = norm.rms_norm(xg, wg, eps).cpu().numpy()
        ref = o.rms_norm(x, w, eps)
        assert (np.abs(y.astype(np.float32) - ref.astype(np.float32)) <= np.spacing(np.abs(ref)).astype(np.float32)).all()
        yx, rx = norm.fused_add_rms_norm(xg, rg, wg, eps)
        assert yx.data_ptr() == xg.data_ptr() and rx.data_ptr() == rg.data_ptr()  # in place
        ref_y, ref_r = o.add_rms_norm(x, r, w, eps)
        assert (rg.cpu().numpy().view(np.uint16) == ref_r.view(np.uint16)).all()
        got = xg.cpu().numpy()
        assert (np.abs(got.astype(np.float32) - ref_y.astype(np.float32))
                <= np.spacing(np.abs(ref_y)).astype(np.float32)).all(), (k, m)


@pytest.mark.gpu
def test_norm_zero_rows_and_errors():
    from tandem_amd.layers import norm

    w = torch.ones(1024, dtype=torch.float16, device="cuda")
    x = torch.zeros(2, 1024, dtype=torch.float16, device="cuda")
    assert (norm.rms_norm(x, w, 1e-6) == 0).all()
    assert norm.rms_norm(x[:0], w, 1e-6).shape == (0, 1024)
    with pytest.raises(RuntimeError, match="K % 512"):
        norm.rms_norm(torch.zeros(1, 1000, dtype=torch.float16, device="cuda"),
                      torch.ones(1000, dtype=torch.float16, device="cuda"), 1e-6)


@pytest.mark.gpu
def test_tiny_decoder_step_matches_oracle():
    model, w = _tiny_model(seed=1)
    for ids in ([7], [3, 999], [1, 2, 3, 4, 5], list(range(20, 44))):
        logits = model.compute_logits(model(torch.tensor(ids, device="cuda")))
        assert logits.shape == (len(ids), TINY.vocab_size) and logits.dtype == torch.float16
        _close(logits, _oracle_step(w, np.array(ids)), 0.02, ids)


@pytest.mark.gpu
def test_fused_norm_step_is_bit_identical(monkeypatch):
    """The step with the norms fused into qkv_proj / gate_up_proj (the default) and with separate
    norm kernels (TANDEM_W4_FUSE_NORM=0) gives the same logits, bit for bit."""
    model, _ = _tiny_model(seed=3)
    for mod in model.modules():  # GEMV entries for M <= 4, where the layer fuses the norm
        if hasattr(mod, "forward_norm"):
            for m in range(1, 5):
                mod.kernels[(mod.out_features, mod.in_features, m)] = ("gemv", 4, 1, 1)
                mod.kernels[(mod.out_features, mod.in_features, m, "silu")] = ("gemv", 8, 1, 1)  # empty slices
    from tandem_amd.layers import w4_hip

    calls = []
    real = w4_hip.W4Extension.w4_decode_norm
    monkeypatch.setattr(w4_hip.W4Extension, "w4_decode_norm", lambda self, *a: calls.append(1) or real(self, *a))
    for ids in ([5], [1, 2, 3], [4, 4, 9, 1], list(range(10, 26))):
        t = torch.tensor(ids, device="cuda")
        calls.clear()
        with torch.inference_mode():
            fused = model.compute_logits(model(t))
            assert len(calls) == (2 * TINY.num_layers if len(ids) <= 4 else 0), (ids, len(calls))
            monkeypatch.setenv("TANDEM_W4_FUSE_NORM", "0")
            separate = model.compute_logits(model(t))
            monkeypatch.delenv("TANDEM_W4_FUSE_NORM")
        assert torch.equal(fused, separate), ids


@pytest.mark.gpu
def test_graph_runner_matches_eager_buckets():
    """Each bucket's replay equals the eager step on the same padded batch, bit for bit, and stays
    so over repeated replays with eager work and synchronisations in between."""
    model, w = _tiny_model(seed=2)
    runner = decode_graph.DecodeGraphRunner(model, max_bs=8, device=torch.device("cuda", 0))
    assert runner.sizes == [1, 2, 4, 8]
    rng = np.random.default_rng(0)
    for rep in range(3):
        for b in (1, 2, 3, 5, 8):
            ids = rng.integers(0, TINY.vocab_size, size=b)
            got = runner.run(ids.tolist()).clone()
            bs = runner.bucket(b)
            padded = torch.zeros(bs, dtype=torch.long, device="cuda")
            padded[:b] = torch.from_numpy(ids).cuda()
            with torch.inference_mode():
                eager = model.compute_logits(model(padded))[:b]
            torch.cuda.synchronize()
            assert torch.equal(got, eager), (rep, b)
            if rep == 0:
                _close(got, _oracle_step(w, ids), 0.02, ("runner", b))
    with pytest.raises(ValueError):
        runner.run(list(range(9)))


def _write_checkpoint(path, cfg: tmodel.DecoderConfig, seed: int):
    """A synthetic AutoAWQ checkpoint of ``cfg`` (separate q/k/v and gate/up tensors, as AutoAWQ
    writes them) and the numpy weights of the step built from it."""
    import json

    from safetensors.torch import save_file

    rng = np.random.default_rng(seed)
    t, w = {}, {"layers": []}
    q, kv = cfg.num_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
    h, inter = cfg.hidden_size, cfg.intermediate_size
    i = 0
    for li in range(cfg.num_layers):
        raw = {}
        for name, (k, n) in (("self_attn.q_proj", (h, q)), ("self_attn.k_proj", (h, kv)), ("self_attn.v_proj", (h, kv)),
                             ("self_attn.o_proj", (q, h)), ("mlp.gate_proj", (h, inter)), ("mlp.up_proj", (h, inter)),
                             ("mlp.down_proj", (inter, h))):
            qw, qz, s, _, _ = o.random_awq(k, n, seed=seed * 100 + i)
            i += 1
            raw[name] = (qw, qz, s)
            for suffix, arr in (("qweight", qw), ("qzeros", qz), ("scales", s)):
                t[f"model.layers.{li}.{name}.{suffix}"] = torch.from_numpy(np.ascontiguousarray(arr))
        n1 = (1.0 + (rng.random(h) - 0.5) * 0.2).astype(np.float16)
        n2 = (1.0 + (rng.random(h) - 0.5) * 0.2).astype(np.float16)
        t[f"model.layers.{li}.input_layernorm.weight"] = torch.from_numpy(n1)
        t[f"model.layers.{li}.post_attention_layernorm.weight"] = torch.from_numpy(n2)
        deq = {k: o.dequant(*v) for k, v in raw.items()}
        w["layers"].append({"qkv": np.concatenate([deq["self_attn.q_proj"], deq["self_attn.k_proj"],
                                                   deq["self_attn.v_proj"]]),
                            "o": deq["self_attn.o_proj"],
                            "gate_up": np.concatenate([deq["mlp.gate_proj"], deq["mlp.up_proj"]]),
                            "down": deq["mlp.down_proj"], "n1": n1, "n2": n2})
    emb = (rng.standard_normal((cfg.vocab_size, h))).astype(np.float16)
    fn = (1.0 + (rng.random(h) - 0.5) * 0.2).astype(np.float16)
    t["model.embed_tokens.weight"] = torch.from_numpy(emb)
    t["model.norm.weight"] = torch.from_numpy(fn)
    save_file(t, str(path / "model.safetensors"))
    (path / "config.json").write_text(json.dumps({"quantization_config": {
        "quant_method": "awq", "bits": 4, "group_size": 128, "zero_point": True, "version": "gemm"}}))
    w.update(emb=emb, head=emb, norm=fn)  # tied embeddings: the logits head is the embedding
    return w


@pytest.mark.gpu
def test_checkpoint_to_graph_runner(tmp_path):
    """AutoAWQ checkpoint -> tandem_amd.loader -> tandem_amd.model (tied embeddings, as Qwen3-1.7B)
    -> bucketed HIP graphs: logits against the oracle's step on the checkpoint's weights."""
    import json

    from tandem_amd import loader

    cfg = tmodel.DecoderConfig(hidden_size=512, intermediate_size=1024, num_heads=4, num_kv_heads=2, head_dim=128,
                               num_layers=2, vocab_size=777, tie_word_embeddings=True)
    w = _write_checkpoint(tmp_path, cfg, seed=5)
    quant = loader.QuantConfig.from_dict(json.loads((tmp_path / "config.json").read_text())["quantization_config"])
    model = tmodel.DecoderModel(cfg, quant)
    loader.load_weights(model, str(tmp_path))
    tmodel.prepare(model, torch.device("cuda", 0), torch.cuda.get_device_name())
    runner = decode_graph.DecodeGraphRunner(model, max_bs=4, device=torch.device("cuda", 0))
    global TINY
    saved, TINY = TINY, cfg  # _oracle_step reads the shapes from TINY
    try:
        for ids in ([3], [776, 0, 5]):
            _close(runner.run(ids), _oracle_step(w, np.array(ids)), 0.02, ("checkpoint", ids))
    finally:
        TINY = saved
