"""Model precision planner: decides, per nn.Linear, who owns it (tfp8 / tbf16 / fp16 / native),
and converts the tfp8 ones to FP8Linear layer by layer (API of tfp8/planner.py:46-139).

The policy -- the name patterns (tfp8/planner.py:20-22), the order in which the rules are tried
and their reason strings (:59-79), and the report() text (:114-126) -- is the reference's, so a
model plans, converts and reports identically.  Here the rules are an ordered table walked once
per Linear; the first rule whose test matches decides the owner.
"""
import re
from collections import Counter
from dataclasses import dataclass

import torch
import torch.nn as nn

from .config import FP8Config
from .linear import FP8Linear

# The reference's patterns, verbatim: they are the policy.
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


@dataclass
class _Ctx:
    name: str
    mod: nn.Module
    domain: str
    config: FP8Config
    tied: set

    @property
    def leaf(self):
        return self.name.rpartition(".")[2]

    @property
    def top(self):
        return self.name.partition(".")[0]


# (test, owner, reason) in the reference's order; owner/reason may depend on the context.
_RULES = (
    (lambda c: bool(getattr(c.mod, "precision_owner", None)),
     lambda c: c.mod.precision_owner, lambda c: "already owned"),
    (lambda c: c.domain == "image" and c.top in _IMAGE_KEEP_COMPONENT,
     lambda c: _IMAGE_KEEP_COMPONENT[c.top], lambda c: f"component '{c.top}' is not quantized in image_safe"),
    (lambda c: id(c.mod.weight) in c.tied,
     lambda c: c.config.fallback, lambda c: "weight shared with another module (tied)"),
    (lambda c: any(re.search(p, c.name) for p in c.config.extra_skip),
     lambda c: c.config.fallback, lambda c: "user skip list"),
    (lambda c: _NEVER.search(c.leaf) is not None,
     lambda c: c.config.fallback, lambda c: f"'{c.leaf}' is precision-sensitive"),
    (lambda c: min(c.mod.out_features, c.mod.in_features) < c.config.min_features,
     lambda c: c.config.fallback, lambda c: f"small Linear (< {c.config.min_features})"),
    (lambda c: c.mod.in_features % 32 != 0,
     lambda c: c.config.fallback, lambda c: "K not a multiple of 32"),
    (lambda c: (_LLM_FP8 if c.domain == "llm" else _IMAGE_FP8).search(c.name) is None,
     lambda c: c.config.fallback, lambda c: "not a recognised large Linear"),
    (lambda c: True, lambda c: "tfp8", lambda c: "large Linear -> FP8 W8A16"),
)


def _tied_parameter_ids(model):
    """ids of parameters that more than one module holds directly (tied weights)."""
    holders = Counter()
    for _, mod in model.named_modules():
        for p in {id(p) for p in mod.parameters(recurse=False)}:
            holders[p] += 1
    return {pid for pid, n in holders.items() if n > 1}


def plan(model: nn.Module, domain: str, config: FP8Config):
    tied = _tied_parameter_ids(model)
    decisions = []
    for name, mod in model.named_modules():
        if isinstance(mod, FP8Linear):
            decisions.append(Decision(name, "FP8Linear", "tfp8", "already converted", ()))
        elif isinstance(mod, nn.Linear):
            ctx = _Ctx(name, mod, domain, config, tied)
            test, owner, reason = next(r for r in _RULES if r[0](ctx))
            decisions.append(Decision(name, type(mod).__name__, owner(ctx), reason(ctx),
                                      (mod.out_features, mod.in_features)))
    return decisions


def prepare_model(model: nn.Module, domain: str = "llm", config: FP8Config | None = None):
    """Quantize, layer by layer, every module the planner assigns to tfp8. Returns the model;
    the plan is attached as `model._tfp8_plan`."""
    if config is None:
        config = FP8Config(profile="llm_safe" if domain == "llm" else "image_safe")
    decisions = plan(model, domain, config)
    for dcs in decisions:
        mod = model.get_submodule(dcs.name)
        if isinstance(mod, FP8Linear):
            continue
        if dcs.owner != "tfp8":
            mod.precision_owner = dcs.owner
            continue
        fp8 = FP8Linear.from_linear(mod, config.fmt, config.weight_group, config.pow2_scale,
                                    large_m=config.large_m, large_m_backend=config.large_m_backend,
                                    workspace_mb=config.workspace_mb, nan_check=config.nan_check,
                                    scale_format=config.scale_format)
        parent, _, leaf = dcs.name.rpartition(".")
        setattr(model.get_submodule(parent) if parent else model, leaf, fp8)
        del mod, fp8
        if torch.cuda.is_available():
            torch.cuda.empty_cache()       # one layer's 16-bit weight at a time is ever resident
    model._tfp8_plan = decisions
    return model


_ROW = "{:48s} {:>14s}  {:6s}  {}"


def report(model, file=None):
    decisions = getattr(model, "_tfp8_plan", [])
    text = [_ROW.format("module", "shape", "owner", "reason")]
    text.extend(_ROW.format(d.name, str(d.shape), d.owner, d.reason) for d in decisions)
    text.append(f"-- {sum(d.owner == 'tfp8' for d in decisions)}/{len(decisions)} Linear modules on tfp8")
    text.extend(f"!! runtime fallback {n}: {m.fallback_reason}" for n, m in model.named_modules()
                if isinstance(m, FP8Linear) and m.fallback is not None)
    out = "\n".join(text)
    print(out, file=file)
    return out


def weight_bytes(model):
    """Bytes held by parameters + buffers, split by dtype (each tensor counted once)."""
    unique = {id(t): t for t in [*model.parameters(), *model.buffers()] if t is not None}
    out = {}
    for t in unique.values():
        key = str(t.dtype).removeprefix("torch.")
        out[key] = out.get(key, 0) + t.numel() * t.element_size()
    return out
