"""FP8Config: conversion policy knobs (API of tfp8/config.py:6-34), plus the scale storage."""
from dataclasses import dataclass, field

PROFILES = ("llm_safe", "image_safe")  # the only profiles the planner commits to


@dataclass
class FP8Config:
    fmt: str = "e4m3fn"
    profile: str = "llm_safe"
    weight_group: int | None = None     # None = per output channel; 32/128 = per-K-group
    activation: str = "fp16"            # W8A16 only
    kv_cache: str = "fp16"
    fallback: str = "tbf16"             # tbf16 | fp16 | native
    min_features: int | None = None     # None -> per-profile default (llm 1024, image 256)
    pow2_scale: bool = True
    large_m: int = 256                  # M at/above which the large-M branch is taken
    large_m_backend: str = "chunked"    # fused | chunked -- both run the fused MFMA GEMM on gfx950
    workspace_mb: int = 32              # kept for API compatibility (no fp16 weight workspace exists)
    nan_check: bool = True              # fall back a module (and log it) on NaN/Inf output
    extra_skip: list[str] = field(default_factory=list)
    scale_format: str = "f32"           # f32 | ue8m0 (power-of-two byte scales)

    def __post_init__(self):
        if self.profile not in PROFILES:
            raise ValueError(f"profile {self.profile!r} not supported; use one of {PROFILES}")
        if self.activation != "fp16":
            raise NotImplementedError("W8A8 is a later phase; only W8A16 is implemented")
        if self.kv_cache != "fp16":
            raise NotImplementedError("FP8 KV cache is a later phase")
        if self.large_m_backend not in ("fused", "chunked"):
            raise ValueError("large_m_backend must be 'fused' or 'chunked'")
        if self.scale_format not in ("f32", "ue8m0"):
            raise ValueError("scale_format must be 'f32' or 'ue8m0'")
        if self.fmt not in ("e4m3fn", "e5m2"):
            raise ValueError(f"unsupported FP8 format {self.fmt!r}")
        if self.min_features is None:
            # LLM projections are wide; DiT/UNet attention and MLP layers are often 256-1024 wide
            # and still worth quantizing (adaLN/time/final modules are excluded by name).
            self.min_features = 1024 if self.profile == "llm_safe" else 256
