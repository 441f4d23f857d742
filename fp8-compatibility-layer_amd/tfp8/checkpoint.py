"""On-disk FP8 checkpoints: a model's FP8Linear layers as native float8 tensors in safetensors.

The reference converts models in memory only (it has no loader, tfp8/README.md:194).  This file
format lets a converted model be stored once and loaded without the 16-bit weights:

    <module>.qweight        float8_e4m3fn / float8_e5m2 [N, K]   the FP8 codes (1 byte each)
    <module>.weight_scale   float32 [N, K/G] or uint8 [N, K/G]    f32 or UE8M0 scales (per-tensor
                                                                  is stored as [N, 1])
    <module>.bias           float32 [N]                           when the layer has a bias
    every other parameter and buffer of the model, under its state_dict name.

Header metadata: "tfp8.format" = "1" and, per FP8Linear, "tfp8.layer.<module>" = JSON with
fmt, group_size, scale_format, out_dtype, in_features, out_features.  Tensors shared by several
names (tied weights) are stored once; "tfp8.alias.<name>" records the name they are stored under.

`load_fp8(model, path)` replaces each listed module (nn.Linear or FP8Linear) with an FP8Linear
built by FP8Linear.from_fp8_checkpoint (tfp8/linear.py:82-98 semantics) and loads the rest.
"""
import json

import torch
import torch.nn as nn

from .linear import FP8Linear

FORMAT_VERSION = "1"
_FP8_DTYPE = {"e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
_DTYPE_NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}
_NAME_DTYPE = {v: k for k, v in _DTYPE_NAME.items()}
_INTERNAL = ("qweight", "weight_scale", "bias_f32")


def _fp8_tensors(name, m):
    q = m.qweight.detach().view(_FP8_DTYPE[m.fmt]).cpu().contiguous()
    out = {f"{name}.qweight": q, f"{name}.weight_scale": m.weight_scale.detach().cpu().contiguous()}
    if m.bias_f32 is not None:
        out[f"{name}.bias"] = m.bias_f32.detach().cpu().contiguous()
    meta = {"fmt": m.fmt, "group_size": m.group_size, "scale_format": m.scale_format,
            "out_dtype": _DTYPE_NAME[m.out_dtype], "in_features": m.in_features, "out_features": m.out_features}
    return out, meta


def save_fp8(model: nn.Module, path: str, metadata: dict | None = None):
    """Write `model` (after prepare_model) to a safetensors file; FP8Linear layers stay 1 byte/weight."""
    from safetensors.torch import save_file

    tensors, meta = {}, {"tfp8.format": FORMAT_VERSION}
    fp8_names = set()
    for name, m in model.named_modules():
        if isinstance(m, FP8Linear):
            t, info = _fp8_tensors(name, m)
            tensors.update(t)
            meta[f"tfp8.layer.{name}"] = json.dumps(info, sort_keys=True)
            fp8_names.add(name)
    stored = {}                                     # storage identity -> name it is stored under
    for key, t in model.state_dict().items():
        owner, _, leaf = key.rpartition(".")
        if owner in fp8_names and leaf in _INTERNAL:
            continue
        ident = (t.untyped_storage().data_ptr(), t.storage_offset(), tuple(t.shape), t.dtype)
        if ident in stored:
            meta[f"tfp8.alias.{key}"] = stored[ident]
            continue
        stored[ident] = key
        tensors[key] = t.detach().cpu().contiguous()
    for k, v in (metadata or {}).items():
        meta[str(k)] = str(v)
    save_file(tensors, path, metadata=meta)


def read_fp8_header(path: str) -> dict:
    """The file's metadata (format version, per-layer descriptions, aliases, user keys)."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        return dict(f.metadata() or {})


def load_fp8(model: nn.Module, path: str, device=None, strict: bool = True, **fp8_kwargs):
    """Load a file written by save_fp8 into `model` (converted or not).  Modules listed as FP8 in the
    file become FP8Linear layers on `device` (default: where the module's parameters are); the other
    tensors are loaded with load_state_dict.  Extra keyword arguments go to FP8Linear (large_m,
    nan_check, ...).  Returns the model."""
    from safetensors.torch import load_file

    meta = read_fp8_header(path)
    if meta.get("tfp8.format") != FORMAT_VERSION:
        raise ValueError(f"{path}: not a tfp8 FP8 checkpoint (format {meta.get('tfp8.format')!r})")
    tensors = load_file(path)
    layers = {k[len("tfp8.layer."):]: json.loads(v) for k, v in meta.items() if k.startswith("tfp8.layer.")}
    for name, info in layers.items():
        old = model.get_submodule(name)
        if not isinstance(old, (nn.Linear, FP8Linear)):
            raise TypeError(f"{name}: expected nn.Linear or FP8Linear, found {type(old).__name__}")
        if (old.in_features, old.out_features) != (info["in_features"], info["out_features"]):
            raise ValueError(f"{name}: shape {(old.out_features, old.in_features)} does not match the file")
        dev = device
        if dev is None:
            p = next(iter(old.buffers() if isinstance(old, FP8Linear) else old.parameters()), None)
            dev = p.device if p is not None else "cpu"
        q = tensors.pop(f"{name}.qweight").to(dev)
        s = tensors.pop(f"{name}.weight_scale").to(dev)
        b = tensors.pop(f"{name}.bias", None)
        kw = dict(fp8_kwargs)
        kw.setdefault("out_dtype", _NAME_DTYPE[info["out_dtype"]])
        new = FP8Linear.from_fp8_checkpoint(q, s, None if b is None else b.to(dev), fmt=info["fmt"], **kw)
        if new.group_size != info["group_size"]:
            raise ValueError(f"{name}: group size {new.group_size} from the scales, file says {info['group_size']}")
        parent, _, leaf = name.rpartition(".")
        setattr(model.get_submodule(parent) if parent else model, leaf, new)
    for key, target in ((k[len("tfp8.alias."):], v) for k, v in meta.items() if k.startswith("tfp8.alias.")):
        tensors[key] = tensors[target]
    missing, unexpected = model.load_state_dict(tensors, strict=False)
    fp8_internal = {f"{n}.{leaf}" for n in layers for leaf in _INTERNAL}
    missing = [k for k in missing if k not in fp8_internal]
    if strict and (missing or unexpected):
        raise KeyError(f"checkpoint mismatch: missing {missing[:8]}, unexpected {list(unexpected)[:8]}")
    return model
