"""Checkpoint loading (checkpoint.py) on the CPU: config parsing, the weight
index, MLX-layout names and shapes -> the model's fused matrices, per-path
quantization overrides, error cases, and save -> load round trips.  No GPU:
the tensors are synthetic codes and scales, and nothing is computed."""

from __future__ import annotations

import importlib
import json

import pytest
import torch

ck = importlib.import_module("mlx-server-runtime_amd.checkpoint")
q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")

QWEN2 = {"model_type": "qwen2", "architectures": ["Qwen2ForCausalLM"], "hidden_size": 128,
         "intermediate_size": 256, "num_attention_heads": 4, "num_key_value_heads": 2,
         "num_hidden_layers": 2, "vocab_size": 64, "rms_norm_eps": 1e-6, "rope_theta": 1e6,
         "tie_word_embeddings": False, "max_position_embeddings": 4096,
         "torch_dtype": "bfloat16", "quantization": {"group_size": 64, "bits": 4}}


def _q(gen, n, k, bits=4, lead=()):
    """Random MLX-layout quantized tensors: codes uint32, bf16 scales/biases."""
    w = torch.randint(0, 2 ** 31 - 1, lead + (n, k * bits // 32), generator=gen,
                      dtype=torch.int64).to(torch.int32).view(torch.uint32)
    s = torch.randn(lead + (n, k // 64), generator=gen).to(torch.bfloat16)
    b = torch.randn(lead + (n, k // 64), generator=gen).to(torch.bfloat16)
    return w, s, b


def _put(sd, path, gen, n, k, bits=4, bias=False, lead=()):
    sd[f"{path}.weight"], sd[f"{path}.scales"], sd[f"{path}.biases"] = _q(gen, n, k, bits, lead)
    if bias:
        sd[f"{path}.bias"] = torch.randn(n, generator=gen).to(torch.bfloat16)


def _state(cfg_payload, moe_layout="stacked", router_bits=4):
    gen = torch.Generator().manual_seed(0)
    c, _ = ck.parse_config(cfg_payload)
    h, d = c.hidden_size, c.head_dim
    sd = {}
    _put(sd, "model.embed_tokens", gen, c.vocab_size, h)
    for i in range(c.num_hidden_layers):
        p = f"model.layers.{i}"
        sd[f"{p}.input_layernorm.weight"] = torch.randn(h, generator=gen).to(torch.bfloat16)
        sd[f"{p}.post_attention_layernorm.weight"] = torch.randn(h, generator=gen).to(
            torch.bfloat16)
        for n, rows in (("q", c.num_attention_heads * d), ("k", c.num_key_value_heads * d),
                        ("v", c.num_key_value_heads * d)):
            _put(sd, f"{p}.self_attn.{n}_proj", gen, rows, h, bias=c.attention_bias)
        _put(sd, f"{p}.self_attn.o_proj", gen, h, c.num_attention_heads * d)
        if c.qk_norm:
            sd[f"{p}.self_attn.q_norm.weight"] = torch.ones(d, dtype=torch.bfloat16)
            sd[f"{p}.self_attn.k_norm.weight"] = torch.ones(d, dtype=torch.bfloat16)
        if c.num_experts:
            E, inter = c.num_experts, c.moe_intermediate_size
            _put(sd, f"{p}.mlp.gate", gen, E, h, bits=router_bits)
            for n, rows, cols in (("gate_proj", inter, h), ("up_proj", inter, h),
                                  ("down_proj", h, inter)):
                if moe_layout == "stacked":
                    _put(sd, f"{p}.mlp.switch_mlp.{n}", gen, rows, cols, lead=(E,))
                else:
                    for e in range(E):
                        _put(sd, f"{p}.mlp.experts.{e}.{n}", gen, rows, cols)
        else:
            _put(sd, f"{p}.mlp.gate_proj", gen, c.intermediate_size, h)
            _put(sd, f"{p}.mlp.up_proj", gen, c.intermediate_size, h)
            _put(sd, f"{p}.mlp.down_proj", gen, h, c.intermediate_size)
    sd["model.norm.weight"] = torch.randn(h, generator=gen).to(torch.bfloat16)
    if not c.tie_word_embeddings:
        _put(sd, "lm_head", gen, c.vocab_size, h)
    return sd


def _write(tmp_path, payload, sd, shards=2):
    from safetensors.torch import save_file
    tmp_path.mkdir(parents=True, exist_ok=True)
    names = list(sd)
    wm = {}
    for i in range(shards):
        part = {n: sd[n] for n in names[i::shards]}
        file = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        save_file(part, str(tmp_path / file))
        wm.update({n: file for n in part})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    (tmp_path / "config.json").write_text(json.dumps(payload))
    return tmp_path


def test_parse_config_variants():
    c, quant = ck.parse_config(QWEN2)
    assert (c.head_dim, c.attention_bias, c.qk_norm, c.num_experts) == (32, True, False, 0)
    assert quant == {"group_size": 64, "bits": 4} and c.bits == 4
    q3 = dict(QWEN2, model_type="qwen3", head_dim=64)
    c3, _ = ck.parse_config(q3)
    assert (c3.head_dim, c3.attention_bias, c3.qk_norm) == (64, False, True)
    moe = dict(q3, model_type="qwen3_moe", num_experts=8, num_experts_per_tok=2,
               moe_intermediate_size=64, norm_topk_prob=True)
    cm, _ = ck.parse_config(moe)
    assert (cm.num_experts, cm.num_experts_per_tok, cm.moe_intermediate_size) == (8, 2, 64)
    no_tie = {k: v for k, v in QWEN2.items() if k != "tie_word_embeddings"}
    assert ck.parse_config(no_tie)[0].tie_word_embeddings  # reference default: tied
    with pytest.raises(ValueError, match="model_type"):
        ck.parse_config(dict(QWEN2, model_type="llama"))
    with pytest.raises(ValueError, match="hidden_size"):
        ck.parse_config({k: v for k, v in QWEN2.items() if k != "hidden_size"})
    with pytest.raises(ValueError, match="head"):
        ck.parse_config(dict(QWEN2, num_key_value_heads=3))


def test_weight_index_errors(tmp_path):
    with pytest.raises(ck.WeightArtifactValidationError, match="missing native weight index"):
        ck.load_weight_index(tmp_path)
    (tmp_path / "model.safetensors.index.json").write_text("{not json")
    with pytest.raises(ck.WeightArtifactValidationError, match="could not parse"):
        ck.load_weight_index(tmp_path)
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {}}))
    with pytest.raises(ck.WeightArtifactValidationError, match="non-empty"):
        ck.load_weight_index(tmp_path)
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {"a": "shard.safetensors"}}))
    with pytest.raises(ck.WeightArtifactValidationError, match="missing native weight files"):
        ck.load_weight_index(tmp_path)


def test_qwen2_names_shapes_and_fusion(tmp_path):
    sd = _state(QWEN2)
    m = ck.load(_write(tmp_path, QWEN2, sd), device="cpu")
    L0 = m.layers[0]
    p = "model.layers.0"
    q, k, v = (sd[f"{p}.self_attn.{n}_proj.weight"].view(torch.int32) for n in "qkv")
    assert torch.equal(L0.qkv.wq, torch.cat([q, k, v]))
    assert torch.equal(L0.qkv.bias, torch.cat([sd[f"{p}.self_attn.{n}_proj.bias"] for n in "qkv"]))
    assert torch.equal(L0.gate_up.scales, torch.cat([sd[f"{p}.mlp.gate_proj.scales"],
                                                     sd[f"{p}.mlp.up_proj.scales"]]))
    assert torch.equal(L0.down.biases, sd[f"{p}.mlp.down_proj.biases"])
    assert torch.equal(m.final_norm, sd["model.norm.weight"])
    assert m.lm_head is not None and m.lm_head.wq.shape == (64, 128 * 4 // 32)
    # save -> load: the same MLX-layout tensors, bit for bit
    out = tmp_path / "resaved"
    ck.save(m, out, shard_bytes=64 * 1024)
    assert len(list(out.glob("*.safetensors"))) > 1
    again = ck.state_dict(ck.load(out, device="cpu"))
    assert set(again) == set(sd)
    for name, t in sd.items():
        assert torch.equal(again[name].view(t.dtype) if t.dtype == torch.uint32 else again[name],
                           t), name


def test_qwen3_moe_layouts_overrides_and_tied_embeddings(tmp_path):
    payload = dict(QWEN2, model_type="qwen3_moe", head_dim=64, num_experts=4,
                   num_experts_per_tok=2, moe_intermediate_size=64, tie_word_embeddings=True)
    payload["quantization"] = {"group_size": 64, "bits": 4,
                               "model.layers.0.mlp.gate": {"group_size": 64, "bits": 8},
                               "model.layers.1.mlp.gate": {"group_size": 64, "bits": 8}}
    stacked = _state(payload, "stacked", router_bits=8)
    m = ck.load(_write(tmp_path / "a", payload, stacked), device="cpu")
    L0 = m.layers[0]
    assert m.lm_head is None and L0.q_norm is not None and L0.moe.gate.bits == 8
    gu = L0.moe.gate_up
    assert gu.wq.shape == (4, 128, 128 * 4 // 32)        # [E, 2 * inter, K * bits / 32]
    sw = "model.layers.0.mlp.switch_mlp"
    assert torch.equal(gu.wq[:, :64], stacked[f"{sw}.gate_proj.weight"].view(torch.int32))
    assert torch.equal(gu.scales[:, 64:], stacked[f"{sw}.up_proj.scales"])
    # the per-expert layout stacks to the same bank
    per = _state(payload, "per_expert", router_bits=8)
    mb = ck.load(_write(tmp_path / "b", payload, per), device="cpu")
    ex = "model.layers.1.mlp.experts"
    assert torch.equal(mb.layers[1].moe.down.wq[2],
                       per[f"{ex}.2.down_proj.weight"].view(torch.int32))
    # round trip through the stacked layout
    out = tmp_path / "c"
    ck.save(m, out)
    again = ck.state_dict(ck.load(out, device="cpu"))
    assert set(again) == set(stacked)


def test_loader_rejects(tmp_path):
    sd = _state(QWEN2)
    bad = dict(sd)
    bad["model.layers.0.mlp.up_proj.scales"] = bad["model.layers.0.mlp.up_proj.scales"].half()
    with pytest.raises(NotImplementedError, match="bfloat16"):
        ck.load(_write(tmp_path / "fp16", QWEN2, bad), device="cpu")
    extra = dict(sd, **{"model.layers.0.mystery.weight": torch.zeros(3)})
    with pytest.raises(ck.WeightArtifactValidationError, match="no place"):
        ck.load(_write(tmp_path / "extra", QWEN2, extra), device="cpu")
    assert ck.load(tmp_path / "extra", device="cpu", strict=False) is not None
    short = {k: v for k, v in sd.items() if k != "model.layers.1.self_attn.o_proj.biases"}
    with pytest.raises(ck.WeightArtifactValidationError, match="o_proj.biases"):
        ck.load(_write(tmp_path / "short", QWEN2, short), device="cpu")
    wide = dict(sd)
    wide["model.layers.0.mlp.down_proj.weight"] = torch.zeros(128, 3, dtype=torch.uint32)
    with pytest.raises(ck.WeightArtifactValidationError, match="codes per row"):
        ck.load(_write(tmp_path / "wide", QWEN2, wide), device="cpu")


def test_parse_config_reference_options():
    """torch_dtype and the RoPE options as the reference reads them
    (models/qwen2.py:261-263,276-277; models/qwen3.py:253-255,356-367)."""
    # no torch_dtype: the reference's KV cache is float16, which this backend does not keep
    with pytest.raises(NotImplementedError, match="float16"):
        ck.parse_config({k: v for k, v in QWEN2.items() if k != "torch_dtype"})
    with pytest.raises(NotImplementedError, match="float16"):
        ck.parse_config(dict(QWEN2, torch_dtype="float16"))
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        ck.parse_config(dict(QWEN2, torch_dtype="float32"))
    assert ck.parse_config(dict(QWEN2, torch_dtype="BFloat16"))[0].hidden_size == 128
    with pytest.raises(NotImplementedError, match="rope_traditional"):
        ck.parse_config(dict(QWEN2, rope_traditional=True))
    assert ck.parse_config(dict(QWEN2, rope_traditional=False))[0].rope_scale == 1.0
    # Qwen3 applies linear RoPE scaling (positions * 1/factor); Qwen2 reads and ignores it
    q3 = dict(QWEN2, model_type="qwen3", head_dim=64)
    lin = {"type": "linear", "factor": 4.0}
    assert ck.parse_config(dict(q3, rope_scaling=lin))[0].rope_scale == 0.25
    assert ck.parse_config(dict(q3, rope_scaling={"rope_type": "default"}))[0].rope_scale == 1.0
    assert ck.parse_config(dict(QWEN2, rope_scaling=lin))[0].rope_scale == 1.0
    with pytest.raises(ValueError, match="unsupported Qwen3 RoPE scaling type"):
        ck.parse_config(dict(q3, rope_scaling={"type": "yarn", "factor": 4.0}))
    with pytest.raises(ValueError, match="positive"):
        ck.parse_config(dict(q3, rope_scaling={"type": "linear", "factor": 0}))
    # the scale reaches the tables: row p is position p * scale
    c = ck.parse_config(dict(q3, rope_scaling=lin))[0]
    cos4, _ = q2.rope_tables(c, 8, "cpu")
    cos1, _ = q2.rope_tables(ck.parse_config(q3)[0], 8, "cpu")
    assert torch.equal(cos4[4], cos1[1])


def _dense(sd, path, gen):
    """Replace a quantized module by an unquantized bfloat16 weight [N, K]."""
    s = sd.pop(f"{path}.scales")
    sd.pop(f"{path}.biases")
    n, k = s.shape[0], s.shape[1] * 64
    sd[f"{path}.weight"] = torch.randn(n, k, generator=gen).to(torch.bfloat16)


def test_unquantized_modules_stay_dense(tmp_path):
    """A module quantized iff its scales are stored (models/qwen2.py:316-324,
    lfm2.py:579-589): lm_head and one o_proj stored in bfloat16 (lm_head also
    marked false per path) load as unquantized linears, unchanged, and save
    back the same; the rest stay quantized."""
    gen = torch.Generator().manual_seed(5)
    payload = dict(QWEN2, quantization={"group_size": 64, "bits": 4, "lm_head": False})
    sd = _state(payload)
    _dense(sd, "lm_head", gen)
    _dense(sd, "model.layers.1.self_attn.o_proj", gen)
    m = ck.load(_write(tmp_path / "a", payload, sd), device="cpu")
    assert isinstance(m.lm_head, q2.DenseLinear)
    assert torch.equal(m.lm_head.weight, sd["lm_head.weight"])
    assert isinstance(m.layers[1].o, q2.DenseLinear) and isinstance(m.layers[0].o, q2.QLinear)
    assert isinstance(m.layers[1].qkv, q2.QLinear)
    ck.save(m, tmp_path / "b")
    again = ck.state_dict(ck.load(tmp_path / "b", device="cpu"))
    assert set(again) == set(sd)
    assert torch.equal(again["lm_head.weight"], sd["lm_head.weight"])
    assert torch.equal(again["model.layers.1.self_attn.o_proj.weight"],
                       sd["model.layers.1.self_attn.o_proj.weight"])
    # no quantization entry at all: every module is an unquantized linear
    plain = {k: v for k, v in payload.items() if k != "quantization"}
    sd2 = _state(QWEN2)
    for name in [n[:-len(".scales")] for n in sd2 if n.endswith(".scales")]:
        _dense(sd2, name, gen)
    m2 = ck.load(_write(tmp_path / "c", plain, sd2), device="cpu")
    assert isinstance(m2.embed, q2.DenseLinear) and isinstance(m2.layers[0].gate_up, q2.DenseLinear)
    assert torch.equal(m2.layers[0].gate_up.weight,
                       torch.cat([sd2["model.layers.0.mlp.gate_proj.weight"],
                                  sd2["model.layers.0.mlp.up_proj.weight"]]))
    # q quantized but k stored dense cannot share one fused q|k|v launch
    sd3 = _state(QWEN2)
    _dense(sd3, "model.layers.0.self_attn.k_proj", gen)
    with pytest.raises(NotImplementedError, match="fused"):
        ck.load(_write(tmp_path / "d", QWEN2, sd3), device="cpu")
    # integer codes without scales are malformed
    sd4 = _state(QWEN2)
    sd4.pop("lm_head.scales")
    sd4.pop("lm_head.biases")
    with pytest.raises(ck.WeightArtifactValidationError, match="without lm_head.scales"):
        ck.load(_write(tmp_path / "e", QWEN2, sd4), device="cpu")
