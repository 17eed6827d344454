"""mlx-community checkpoints without MLX: safetensors in, a Qwen2Model out.

Restates the reference's loading path for the quantized models
(python/mlx_worker/native_mlx/mapping.py:61-139 load_mapped_weights /
load_weight_index; models/qwen2.py:231-327 parse_qwen2_config,
Qwen2WeightAdapter, build_qwen2_model; models/qwen3.py for head_dim and the
q/k norms; models/lfm2.py:569-591 for per-path quantization overrides):

* the weight index is `model.safetensors.index.json` (`weight_map`: tensor
  name -> shard file), or a single `model.safetensors`;
* a module is quantized iff the checkpoint holds `{path}.scales`
  (qwen2.py:316-324); its (group_size, bits) are config["quantization"]'s,
  or that dict's entry for the module path (lfm2.py:584-586);
* quantized tensors keep MLX's layout: `{path}.weight` uint32
  [N, K*bits/32], `{path}.scales` / `{path}.biases` [N, K/group_size];
  mixture-of-experts banks are stacked per expert,
  `mlp.switch_mlp.{gate,up,down}_proj.*` [E, N, ...] (or per-expert
  `mlp.experts.{e}.*`, stacked on load); codes at 2, 3, 5 or 6 bits stay
  packed in linear layers (one-row matmuls read them at their width, larger
  ones rewrite them one byte each per call) and are rewritten one byte each
  once, on a GPU device, in expert banks (the gather kernels read 4- and
  8-bit codes; same scales and biases: the same dequantized weights).

Tensors are read with safetensors (no pickle), straight to the target device.
Modules stored without `{path}.scales` (and every module of a checkpoint
with no `quantization` entry) stay unquantized bfloat16 linears, as the
reference's class_predicate leaves them; expert banks must be quantized.
Scales and biases must be bfloat16 (the kernels' type); a float16 checkpoint
raises NotImplementedError rather than silently rounding its scales, and so
do configs this backend cannot run as the reference would (a float16 KV
cache, rope_traditional).

`save` writes a model back in the same layout (used to round-trip the
loader in the tests).
"""

from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Any

import torch

from . import core
from .moe import MoEBlock, QExperts
from .qwen2 import DenseLinear, Layer, QLinear, Qwen2Config, Qwen2Model, _concat


class WeightArtifactValidationError(ValueError):
    """Checkpoint files missing or malformed (mapping.py:13-14)."""


# ---------------------------------------------------------------- config
def parse_config(payload: dict[str, Any]) -> tuple[Qwen2Config, dict | None]:
    """config.json -> (Qwen2Config, quantization dict or None); model_type qwen2,
    qwen3 or qwen3_moe (checks as parse_qwen2_config, qwen2.py:231-282)."""
    mt = payload.get("model_type")
    if mt not in ("qwen2", "qwen3", "qwen3_moe"):
        raise ValueError(f"unsupported model_type {mt!r} (qwen2, qwen3, qwen3_moe)")
    required = ("hidden_size", "intermediate_size", "num_attention_heads",
                "num_hidden_layers", "vocab_size", "rms_norm_eps")
    for name in required:
        if not isinstance(payload.get(name), (int, float)):
            raise ValueError(f"missing or invalid {name}")
    heads = int(payload["num_attention_heads"])
    kv_heads = int(payload.get("num_key_value_heads", heads))
    hidden = int(payload["hidden_size"])
    head_dim = int(payload.get("head_dim") or hidden // heads)
    if heads % kv_heads or (mt == "qwen2" and hidden % heads):
        raise ValueError("invalid head dimensions")
    # The reference's paged KV cache takes the checkpoint's dtype (float16 when
    # the config names none, qwen2.py:261-263, qwen3.py:253-255); the
    # kernels here keep a bfloat16 cache, so only bfloat16 loads.
    kv_dtype = str(payload.get("torch_dtype", "float16")).lower()
    if kv_dtype not in ("float16", "bfloat16"):
        raise ValueError("native paged KV requires float16 or bfloat16 torch_dtype")
    if kv_dtype != "bfloat16":
        raise NotImplementedError(
            f"torch_dtype {kv_dtype}: this backend keeps a bfloat16 paged KV cache")
    if payload.get("rope_traditional", False):  # qwen2.py:64,276
        raise NotImplementedError("rope_traditional=True: this backend implements the "
                                  "non-traditional (rotate-half) RoPE only")
    rope_scale = _rope_scale(payload.get("rope_scaling")) if mt != "qwen2" else 1.0
    quant = payload.get("quantization") or payload.get("quantization_config")
    group_size = int(quant["group_size"]) if quant else 64
    bits = int(quant["bits"]) if quant else 4
    moe = mt == "qwen3_moe"
    cfg = Qwen2Config(
        hidden_size=hidden, intermediate_size=int(payload["intermediate_size"]),
        num_attention_heads=heads, num_key_value_heads=kv_heads,
        num_hidden_layers=int(payload["num_hidden_layers"]),
        vocab_size=int(payload["vocab_size"]), rms_norm_eps=float(payload["rms_norm_eps"]),
        rope_theta=float(payload.get("rope_theta", 1_000_000.0)), rope_scale=rope_scale,
        tie_word_embeddings=bool(payload.get("tie_word_embeddings", True)),
        group_size=group_size, bits=bits,
        head_dim_=head_dim if head_dim != hidden // heads else 0,
        attention_bias=bool(payload.get("attention_bias", mt == "qwen2")),
        qk_norm=mt != "qwen2",
        num_experts=int(payload.get("num_experts", 0)) if moe else 0,
        num_experts_per_tok=int(payload.get("num_experts_per_tok", 0)) if moe else 0,
        moe_intermediate_size=int(payload.get("moe_intermediate_size", 0)) if moe else 0,
        norm_topk_prob=bool(payload.get("norm_topk_prob", True)))
    return cfg, quant


def _rope_scale(rope_scaling: dict[str, Any] | None) -> float:
    """Position scale of Qwen3's RoPE (models/qwen3.py:356-367): 1/factor for
    "linear" scaling, 1 for none or "default", anything else rejected.  The
    reference's Qwen2 reads rope_scaling but never applies it
    (models/qwen2.py:62-66)."""
    if not rope_scaling:
        return 1.0
    rope_type = rope_scaling.get("type") or rope_scaling.get("rope_type")
    if rope_type == "linear":
        factor = float(rope_scaling.get("factor", 1.0))
        if factor <= 0:
            raise ValueError("Qwen3 rope scaling factor must be positive")
        return 1.0 / factor
    if rope_type in (None, "default"):
        return 1.0
    raise ValueError(f"unsupported Qwen3 RoPE scaling type: {rope_type}")


# ---------------------------------------------------------------- index
def load_weight_index(model_path: str | os.PathLike) -> dict[str, str]:
    """Tensor name -> shard file (mapping.py:85-139)."""
    root = Path(model_path)
    index_path = root / "model.safetensors.index.json"
    if index_path.exists():
        name = index_path.name
        try:
            payload = json.loads(index_path.read_text())
        except (OSError, json.JSONDecodeError) as exc:
            raise WeightArtifactValidationError(f"could not parse {name}: {exc}") from exc
        weight_map = payload.get("weight_map")
        if not isinstance(weight_map, dict) or not weight_map:
            raise WeightArtifactValidationError(f"{name} is missing non-empty weight_map")
        if any(not isinstance(k, str) or not isinstance(v, str) for k, v in weight_map.items()):
            raise WeightArtifactValidationError(f"{name} contains non-string weight entries")
        missing = sorted({v for v in weight_map.values() if not (root / v).exists()})
        if missing:
            raise WeightArtifactValidationError(
                "missing native weight files: " + ", ".join(missing))
        return dict(weight_map)
    single = root / "model.safetensors"
    if single.exists():
        from safetensors import safe_open
        with safe_open(str(single), framework="pt", device="cpu") as f:
            return {k: single.name for k in f.keys()}
    raise WeightArtifactValidationError(f"missing native weight index: {index_path.name}")


def read_tensors(model_path, weight_map: dict[str, str], device) -> dict[str, torch.Tensor]:
    """Every tensor of the index, loaded per shard straight to `device`."""
    from safetensors import safe_open
    root = Path(model_path)
    by_file: dict[str, list[str]] = {}
    for name, file in weight_map.items():
        by_file.setdefault(file, []).append(name)
    out = {}
    for file, names in by_file.items():
        try:
            with safe_open(str(root / file), framework="pt", device=str(device)) as f:
                present = set(f.keys())
                for name in names:
                    if name not in present:
                        raise WeightArtifactValidationError(f"missing tensor {name!r} in {file}")
                    out[name] = f.get_tensor(name)
        except WeightArtifactValidationError:
            raise
        except Exception as exc:  # noqa: BLE001 -- report any reader failure as the reference does
            raise WeightArtifactValidationError(
                f"could not load native weights from {file}: {exc}") from exc
    return out


# ---------------------------------------------------------------- modules
class _Builder:
    def __init__(self, tensors, cfg: Qwen2Config, quant: dict | None, device):
        self.t, self.cfg, self.quant, self.device = tensors, cfg, quant or {}, device
        self.used: set[str] = set()

    def has(self, name: str) -> bool:
        return name in self.t

    def take(self, name: str) -> torch.Tensor:
        if name not in self.t:
            raise WeightArtifactValidationError(f"missing tensor {name!r}")
        self.used.add(name)
        return self.t[name]

    def params(self, path: str) -> tuple[int, int]:
        over = self.quant.get(path)
        src = over if isinstance(over, dict) else self.quant
        return int(src.get("group_size", self.cfg.group_size)), int(src.get("bits", self.cfg.bits))

    def _bf16(self, name: str, t: torch.Tensor) -> torch.Tensor:
        if t.dtype != torch.bfloat16:
            raise NotImplementedError(
                f"{name} is {t.dtype}: this backend computes with bfloat16 scales and biases")
        return t.contiguous()

    def norm(self, path: str) -> torch.Tensor:
        return self.take(f"{path}.weight").to(torch.bfloat16).contiguous()

    def linear(self, path: str) -> QLinear | DenseLinear:
        """{path}.* -> QLinear when the checkpoint holds {path}.scales (with the
        config's or the path's own group size and bits, lfm2.py:579-589), else
        an unquantized DenseLinear, as the reference's class_predicate leaves
        such a module (qwen2.py:316-324)."""
        bias = self.take(f"{path}.bias").to(torch.bfloat16) if self.has(f"{path}.bias") else None
        if not self.quant or not self.has(f"{path}.scales"):
            w = self.take(f"{path}.weight")
            if not w.is_floating_point():
                raise WeightArtifactValidationError(
                    f"{path}: integer weight {tuple(w.shape)} without {path}.scales")
            return DenseLinear(w.to(torch.bfloat16), bias)
        gs, bits = self.params(path)
        wq = self.take(f"{path}.weight")
        s = self._bf16(f"{path}.scales", self.take(f"{path}.scales"))
        b = self._bf16(f"{path}.biases", self.take(f"{path}.biases"))
        K = s.shape[-1] * gs
        if wq.shape[-1] * 32 != K * bits:
            raise WeightArtifactValidationError(
                f"{path}: weight {tuple(wq.shape)} does not hold {K} {bits}-bit codes per row")
        wq = wq.view(torch.int32) if wq.dtype == torch.uint32 else wq
        return QLinear(wq.contiguous(), s, b, bias, gs, bits)

    def experts(self, path: str, proj: str) -> QExperts:
        stacked = f"{path}.switch_mlp.{proj}"
        is_stacked = self.has(f"{stacked}.weight")
        if is_stacked:
            ql = self.linear(stacked)
            parts = [ql]
        else:
            E = self.cfg.num_experts
            parts = [self.linear(f"{path}.experts.{e}.{proj}") for e in range(E)]
        if not all(isinstance(p, QLinear) for p in parts):
            raise NotImplementedError(f"{path}.{proj}: unquantized experts (this backend runs "
                                      "the experts through gather_qmm only)")
        if not is_stacked:
            ql = QLinear(torch.stack([p.wq for p in parts]), torch.stack([p.scales for p in parts]),
                         torch.stack([p.biases for p in parts]), None, parts[0].group_size,
                         parts[0].bits)
        wq, bits = ql.wq, ql.bits
        if bits not in (4, 8) and wq.is_cuda:
            # the gather kernels read 4- and 8-bit codes: a 2/3/5/6-bit bank is
            # rewritten one byte each, once here
            wq, bits = core.repack_codes_u8(wq.contiguous(), bits), 8
        return QExperts(wq, ql.scales, ql.biases, ql.group_size, bits)


def _qparams(ql) -> tuple[int, int] | None:
    """(group_size, bits) of a quantized linear, None for an unquantized one."""
    return (ql.group_size, ql.bits) if isinstance(ql, QLinear) else None


def _fuse_experts(a: QExperts, b: QExperts) -> QExperts:
    if (a.group_size, a.bits) != (b.group_size, b.bits):
        raise NotImplementedError("gate and up experts quantized differently")
    return QExperts(torch.cat([a.wq, b.wq], 1), torch.cat([a.scales, b.scales], 1),
                    torch.cat([a.biases, b.biases], 1), a.group_size, a.bits)


def build_model(cfg: Qwen2Config, tensors: dict[str, torch.Tensor], quant: dict | None,
                device, strict: bool = True) -> Qwen2Model:
    """Canonical names (qwen2.py:331-340) -> Qwen2Model with fused q|k|v and gate|up."""
    bld = _Builder(tensors, cfg, quant, device)
    embed = bld.linear("model.embed_tokens")
    layers = []
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}"
        parts = [bld.linear(f"{p}.self_attn.{n}_proj") for n in ("q", "k", "v")]
        if len({_qparams(q) for q in parts}) != 1:
            raise NotImplementedError(f"{p}: q/k/v quantized differently cannot be fused")
        layer = Layer(bld.norm(f"{p}.input_layernorm"), bld.norm(f"{p}.post_attention_layernorm"),
                      _concat(parts), bld.linear(f"{p}.self_attn.o_proj"))
        if cfg.qk_norm:
            layer.q_norm = bld.norm(f"{p}.self_attn.q_norm")
            layer.k_norm = bld.norm(f"{p}.self_attn.k_norm")
        if cfg.num_experts:
            gate_up = _fuse_experts(bld.experts(f"{p}.mlp", "gate_proj"),
                                    bld.experts(f"{p}.mlp", "up_proj"))
            layer.moe = MoEBlock(bld.linear(f"{p}.mlp.gate"), gate_up,
                                 bld.experts(f"{p}.mlp", "down_proj"), cfg.num_experts_per_tok,
                                 cfg.norm_topk_prob)
        else:
            gate, up = bld.linear(f"{p}.mlp.gate_proj"), bld.linear(f"{p}.mlp.up_proj")
            if _qparams(gate) != _qparams(up):
                raise NotImplementedError(f"{p}: gate/up quantized differently cannot be fused")
            layer.gate_up = _concat([gate, up])
            layer.down = bld.linear(f"{p}.mlp.down_proj")
        layers.append(layer)
    final_norm = bld.norm("model.norm")
    lm_head = None if cfg.tie_word_embeddings else bld.linear("lm_head")
    if strict:
        unused = sorted(set(tensors) - bld.used)
        if unused:  # model.load_weights(weights, strict=True), qwen2.py:325
            raise WeightArtifactValidationError(
                f"{len(unused)} checkpoint tensors have no place in the model, e.g. {unused[:3]}")
    return Qwen2Model(cfg, embed, layers, final_norm, lm_head)


def load(model_path: str | os.PathLike, device="cuda:0", strict: bool = True) -> Qwen2Model:
    """config.json + safetensors shards -> Qwen2Model on `device`."""
    root = Path(model_path)
    try:
        payload = json.loads((root / "config.json").read_text())
    except (OSError, json.JSONDecodeError) as exc:
        raise WeightArtifactValidationError(f"could not parse config.json: {exc}") from exc
    cfg, quant = parse_config(payload)
    tensors = read_tensors(root, load_weight_index(root), device)
    return build_model(cfg, tensors, quant, device, strict)


# ---------------------------------------------------------------- save
def _split_rows(ql, sizes: list[int]) -> list:
    out, r = [], 0
    for n in sizes:
        if isinstance(ql, DenseLinear):
            out.append(DenseLinear(ql.weight[r:r + n],
                                   None if ql.bias is None else ql.bias[r:r + n]))
            r += n
            continue
        out.append(QLinear(ql.wq[r:r + n], ql.scales[r:r + n], ql.biases[r:r + n],
                           None if ql.bias is None else ql.bias[r:r + n], ql.group_size, ql.bits))
        r += n
    return out


def _export(model: Qwen2Model) -> tuple[dict[str, torch.Tensor], dict[str, dict]]:
    """MLX-layout tensors of `model` (the inverse of build_model), on the CPU, and
    the per-path quantization overrides of modules whose (group_size, bits)
    differ from the config's."""
    c = model.cfg
    d = c.head_dim
    sd: dict[str, torch.Tensor] = {}
    overrides: dict[str, dict] = {}

    def put(path, ql, gs=None, bits=None):
        if isinstance(ql, DenseLinear):  # stored unquantized: no scales, no override
            sd[f"{path}.weight"] = ql.weight
            if ql.bias is not None:
                sd[f"{path}.bias"] = ql.bias
            return
        gs = gs or getattr(ql, "group_size", c.group_size)
        bits = bits or getattr(ql, "bits", c.bits)
        if (gs, bits) != (c.group_size, c.bits):
            overrides[path] = {"group_size": gs, "bits": bits}
        sd[f"{path}.weight"] = ql.wq.view(torch.uint32)
        sd[f"{path}.scales"], sd[f"{path}.biases"] = ql.scales, ql.biases
        if getattr(ql, "bias", None) is not None:
            sd[f"{path}.bias"] = ql.bias

    put("model.embed_tokens", model.embed)
    for i, layer in enumerate(model.layers):
        p = f"model.layers.{i}"
        sd[f"{p}.input_layernorm.weight"] = layer.input_norm
        sd[f"{p}.post_attention_layernorm.weight"] = layer.post_norm
        q, k, v = _split_rows(layer.qkv, [c.num_attention_heads * d, c.num_key_value_heads * d,
                                          c.num_key_value_heads * d])
        for n, ql in zip(("q", "k", "v"), (q, k, v)):
            put(f"{p}.self_attn.{n}_proj", ql)
        put(f"{p}.self_attn.o_proj", layer.o)
        if layer.q_norm is not None:
            sd[f"{p}.self_attn.q_norm.weight"] = layer.q_norm
            sd[f"{p}.self_attn.k_norm.weight"] = layer.k_norm
        if layer.moe is not None:
            m = layer.moe
            put(f"{p}.mlp.gate", m.gate)
            inter = m.down.wq.shape[-1] * 32 // m.down.bits
            gu = m.gate_up
            for n, sl in (("gate_proj", slice(0, inter)), ("up_proj", slice(inter, 2 * inter))):
                put(f"{p}.mlp.switch_mlp.{n}",
                    QLinear(gu.wq[:, sl], gu.scales[:, sl], gu.biases[:, sl], None,
                            gu.group_size, gu.bits))
            put(f"{p}.mlp.switch_mlp.down_proj",
                QLinear(m.down.wq, m.down.scales, m.down.biases, None, m.down.group_size,
                        m.down.bits))
        else:
            gate, up = _split_rows(layer.gate_up, [c.intermediate_size] * 2)
            put(f"{p}.mlp.gate_proj", gate)
            put(f"{p}.mlp.up_proj", up)
            put(f"{p}.mlp.down_proj", layer.down)
    sd["model.norm.weight"] = model.final_norm
    if model.lm_head is not None:
        put("lm_head", model.lm_head)
    return {k: v.detach().contiguous().cpu() for k, v in sd.items()}, overrides


def state_dict(model: Qwen2Model) -> dict[str, torch.Tensor]:
    """MLX-layout tensors of `model` (the inverse of build_model), on the CPU."""
    return _export(model)[0]


def config_payload(cfg: Qwen2Config, overrides: dict[str, dict] | None = None) -> dict[str, Any]:
    """config.json for `cfg` (Hugging Face names, MLX's quantization entry)."""
    mt = "qwen3_moe" if cfg.num_experts else ("qwen3" if cfg.qk_norm else "qwen2")
    out = {"model_type": mt, "architectures": [{"qwen2": "Qwen2ForCausalLM",
                                                "qwen3": "Qwen3ForCausalLM",
                                                "qwen3_moe": "Qwen3MoeForCausalLM"}[mt]],
           "hidden_size": cfg.hidden_size, "intermediate_size": cfg.intermediate_size,
           "num_attention_heads": cfg.num_attention_heads,
           "num_key_value_heads": cfg.num_key_value_heads,
           "num_hidden_layers": cfg.num_hidden_layers, "vocab_size": cfg.vocab_size,
           "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta,
           "tie_word_embeddings": cfg.tie_word_embeddings, "head_dim": cfg.head_dim,
           "attention_bias": cfg.attention_bias, "max_position_embeddings": 32768,
           "torch_dtype": "bfloat16",
           "quantization": {"group_size": cfg.group_size, "bits": cfg.bits, **(overrides or {})}}
    if cfg.rope_scale != 1.0:
        out["rope_scaling"] = {"type": "linear", "factor": 1.0 / cfg.rope_scale}
    if cfg.num_experts:
        out.update(num_experts=cfg.num_experts, num_experts_per_tok=cfg.num_experts_per_tok,
                   moe_intermediate_size=cfg.moe_intermediate_size,
                   norm_topk_prob=cfg.norm_topk_prob)
    return out


def save(model: Qwen2Model, model_path: str | os.PathLike, shard_bytes: int = 1 << 30) -> None:
    """Write config.json, model-0000i-of-0000n.safetensors shards and the index."""
    from safetensors.torch import save_file
    root = Path(model_path)
    root.mkdir(parents=True, exist_ok=True)
    sd, overrides = _export(model)
    shards: list[dict[str, torch.Tensor]] = [{}]
    size = 0
    for name, t in sd.items():
        nb = t.numel() * t.element_size()
        if shards[-1] and size + nb > shard_bytes:
            shards.append({})
            size = 0
        shards[-1][name] = t
        size += nb
    weight_map = {}
    for i, shard in enumerate(shards):
        file = f"model-{i + 1:05d}-of-{len(shards):05d}.safetensors"
        save_file(shard, str(root / file), metadata={"format": "mlx"})
        weight_map.update({name: file for name in shard})
    (root / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": {}, "weight_map": weight_map}, indent=1))
    (root / "config.json").write_text(json.dumps(config_payload(model.cfg, overrides), indent=1))


__all__ = ["WeightArtifactValidationError", "parse_config", "load_weight_index", "read_tensors",
           "build_model", "load", "state_dict", "config_payload", "save"]
