"""Model precision planner: decides, per nn.Linear, who owns it (tfp8 / tbf16 / fp16 / native),
and converts the tfp8 ones to FP8Linear layer by layer (API of tfp8/planner.py:46-139).

The policy (name patterns, order of the rules, reason strings) is the reference's, so a model
plans identically; see tfp8/planner.py:20-22 for the patterns and :59-79 for the rules.
"""
import re
from dataclasses import dataclass

import torch
import torch.nn as nn

from .config import FP8Config
from .linear import FP8Linear

# Same patterns as tfp8/planner.py:20-22 (they are the policy, so they must match exactly).
_LLM_FP8 = re.compile(r"(q_proj|k_proj|v_proj|o_proj|qkv|out_proj|gate_proj|up_proj|down_proj|fc1|fc2|w1|w2|w3|mlp)")
_IMAGE_FP8 = re.compile(r"(to_q|to_k|to_v|to_out|qkv|proj|attn|ff|mlp|fc1|fc2|linear)")
_NEVER = re.compile(r"(lm_head|embed|router|gate$|gating|lora|adapter|norm|time|t_embed|adaln|ada_ln|modulation"
                    r"|final|proj_out|head$)", re.I)
_IMAGE_KEEP_COMPONENT = {"vae": "fp16", "text_encoder": "tbf16", "text_encoder_2": "tbf16"}


@dataclass
class Decision:
    name: str
    kind: str
    owner: str          # tfp8 | tbf16 | fp16 | native
    reason: str
    shape: tuple = ()


def _shared_param_ids(model):
    """ids of parameters reachable from more than one module (tied weights)."""
    owner, shared = {}, set()
    for mod_name, mod in model.named_modules():
        for _, p in mod.named_parameters(recurse=False):
            first = owner.setdefault(id(p), mod_name)
            if first != mod_name:
                shared.add(id(p))
    return shared


def _rule(name, mod, domain, config, shared):
    """(owner, reason) for one nn.Linear, first matching rule wins."""
    leaf = name.split(".")[-1]
    top = name.split(".")[0]
    shape = (mod.out_features, mod.in_features)
    if getattr(mod, "precision_owner", None):
        return mod.precision_owner, "already owned"
    if domain == "image" and top in _IMAGE_KEEP_COMPONENT:
        return _IMAGE_KEEP_COMPONENT[top], f"component '{top}' is not quantized in image_safe"
    if id(mod.weight) in shared:
        return config.fallback, "weight shared with another module (tied)"
    if any(re.search(p, name) for p in config.extra_skip):
        return config.fallback, "user skip list"
    if _NEVER.search(leaf):
        return config.fallback, f"'{leaf}' is precision-sensitive"
    if min(shape) < config.min_features:
        return config.fallback, f"small Linear (< {config.min_features})"
    if mod.in_features % 32:
        return config.fallback, "K not a multiple of 32"
    if not (_LLM_FP8 if domain == "llm" else _IMAGE_FP8).search(name):
        return config.fallback, "not a recognised large Linear"
    return "tfp8", "large Linear -> FP8 W8A16"


def plan(model: nn.Module, domain: str, config: FP8Config):
    shared = _shared_param_ids(model)
    out = []
    for name, mod in model.named_modules():
        if isinstance(mod, FP8Linear):
            out.append(Decision(name, "FP8Linear", "tfp8", "already converted", ()))
        elif isinstance(mod, nn.Linear):
            owner, reason = _rule(name, mod, domain, config, shared)
            out.append(Decision(name, type(mod).__name__, owner, reason, (mod.out_features, mod.in_features)))
    return out


def _set_submodule(root, name, new):
    *path, leaf = name.split(".")
    parent = root
    for p in path:
        parent = getattr(parent, p)
    setattr(parent, leaf, new)


def prepare_model(model: nn.Module, domain: str = "llm", config: FP8Config | None = None):
    """Quantize, layer by layer, every module the planner assigns to tfp8. Returns the model;
    the plan is attached as `model._tfp8_plan`."""
    config = config or FP8Config(profile="llm_safe" if domain == "llm" else "image_safe")
    decisions = plan(model, domain, config)
    mods = dict(model.named_modules())
    for dcs in decisions:
        mod = mods[dcs.name]
        if isinstance(mod, FP8Linear):
            continue
        if dcs.owner == "tfp8":
            new = FP8Linear.from_linear(mod, config.fmt, config.weight_group, config.pow2_scale,
                                        large_m=config.large_m, large_m_backend=config.large_m_backend,
                                        workspace_mb=config.workspace_mb, nan_check=config.nan_check,
                                        scale_format=config.scale_format)
            _set_submodule(model, dcs.name, new)
            del mod
            if torch.cuda.is_available():
                torch.cuda.empty_cache()
        else:
            mod.precision_owner = dcs.owner
    model._tfp8_plan = decisions
    return model


def report(model, file=None):
    rows = getattr(model, "_tfp8_plan", [])
    lines = [f"{'module':48s} {'shape':>14s}  {'owner':6s}  reason"]
    lines += [f"{r.name:48s} {str(r.shape):>14s}  {r.owner:6s}  {r.reason}" for r in rows]
    lines.append(f"-- {sum(r.owner == 'tfp8' for r in rows)}/{len(rows)} Linear modules on tfp8")
    for name, m in model.named_modules():
        if isinstance(m, FP8Linear) and m.fallback is not None:
            lines.append(f"!! runtime fallback {name}: {m.fallback_reason}")
    text = "\n".join(lines)
    print(text, file=file)
    return text


def weight_bytes(model):
    """Bytes held by parameters + buffers, split by dtype."""
    out, seen = {}, set()
    for t in list(model.parameters()) + list(model.buffers()):
        if t is None or id(t) in seen:
            continue
        seen.add(id(t))
        k = str(t.dtype).replace("torch.", "")
        out[k] = out.get(k, 0) + t.numel() * t.element_size()
    return out
