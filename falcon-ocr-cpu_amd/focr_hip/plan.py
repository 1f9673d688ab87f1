"""Prefill plans and their labels on the `hip` backend.

The reference picks a prefill projection and attention kernel per body and
CPU (``prefill_plan``, src/kernels/mod.rs:185-259) and records their labels
(``Display`` of ``PrefillProjection`` / ``PrefillAttention``,
src/kernels/mod.rs:156-180) in every page record's plan; ``--resume``
compares them (``Kernels::from_plan``, src/book/resume.rs:102-137). The `hip`
backend adds its own kernels under their own labels, so a resumed run never
mixes CPU and GPU records silently:

    projection  hip-f32-split | hip-f32-mfma | hip-f32-chain | hip-i16
    attention   hip | hip-static | hip-bf16 | hip-bf16-static

``hip_prefill_plan`` applies the reference's predicate set with the GPU's
kernels: an 8-bit body whose matrices the INT16 panels hold takes the INT16
projections (bitwise the reference's INT16 panels) unless the tuning asks for
FP32 ones; other quantized bodies take the bitwise FP32 chain
(PanelAvx2's order); an FP32 body takes FP32 products from power-of-two
scaled FP16 pairs on the FP16 matrix cores (the reference's ``gemm`` crate order is not
reproduced bitwise by any kernel; this one is the fastest within the FP32
tolerance; ``hip-f32-mfma``, the FP32 matrix cores, stays a valid label).
Attention: an 8-bit body takes BF16 attention unless ``prefill_bf16`` is off
(static softmax when ``prefill_softmax`` asks for it); FP32 tiles take the
static softmax for 16-bit bodies (or when ``prefill_softmax_fp32`` asks for
it on a quantized body), the online one otherwise.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

from . import ExpMode, FocrError, PrefillProjection, Softmax

PROJECTION_LABELS = {PrefillProjection.F32_MFMA: "hip-f32-mfma", PrefillProjection.F32_CHAIN: "hip-f32-chain",
                     PrefillProjection.I16: "hip-i16", PrefillProjection.F32_SPLIT: "hip-f32-split"}
ATTENTION_KINDS = ("hip", "hip-static", "hip-bf16", "hip-bf16-static")


@dataclass(frozen=True)
class HipPrefillPlan:
    projection: PrefillProjection
    attention: str  # one of ATTENTION_KINDS

    def labels(self) -> dict:
        """The plan's `prefill` object as a page record stores it."""
        return {"projection": PROJECTION_LABELS[self.projection], "attention": self.attention}

    @staticmethod
    def from_labels(value: dict) -> "HipPrefillPlan":
        proj = {v: k for k, v in PROJECTION_LABELS.items()}.get(value.get("projection"))
        att = value.get("attention")
        if proj is None or att not in ATTENTION_KINDS:
            raise FocrError(-1, f"not a hip prefill plan: {value}")
        return HipPrefillPlan(proj, att)

    def bf16(self) -> bool:
        return self.attention.startswith("hip-bf16")

    def softmax(self) -> Softmax:
        """The softmax the plan's attention kernel runs."""
        return Softmax.STATIC if self.attention.endswith("-static") else Softmax.ONLINE


def hip_prefill_plan(body_bits: Optional[int], i16_misfit: bool, prefill_bf16: bool = True,
                     prefill_softmax: str = "static", prefill_softmax_fp32: Optional[str] = None,
                     prefill_projections: str = "i16") -> HipPrefillPlan:
    """The `hip` plan for a body of `body_bits` (None: FP32), mirroring
    prefill_plan's predicates (src/kernels/mod.rs:203-259). The knobs take the
    reference's `--tune` values and defaults (src/config/tuning.rs:60-130):
    prefill_bf16 on ("attention"), prefill_softmax "static",
    prefill_softmax_fp32 unset, prefill_projections "i16" (or "fp32")."""
    for name, v, allowed in (("prefill_softmax", prefill_softmax, ("online", "static")),
                             ("prefill_softmax_fp32", prefill_softmax_fp32, (None, "online", "static")),
                             ("prefill_projections", prefill_projections, ("i16", "fp32"))):
        if v not in allowed:
            raise FocrError(-1, f"{name}: {v!r}")
    if body_bits not in (None, 8, 16):
        raise FocrError(-1, "body_bits: None (FP32), 8 or 16")
    panel = body_bits is not None
    fp32_softmax = prefill_softmax_fp32 or ("static" if body_bits == 16 else "online")
    static_fp32 = panel and fp32_softmax == "static"
    if not panel:
        projection = PrefillProjection.F32_SPLIT
    elif body_bits == 8 and not i16_misfit and prefill_projections == "i16":
        projection = PrefillProjection.I16
    else:
        projection = PrefillProjection.F32_CHAIN
    if panel and body_bits == 8 and prefill_bf16:
        attention = "hip-bf16-static" if prefill_softmax == "static" else "hip-bf16"
    else:
        attention = "hip-static" if static_fp32 else "hip"
    return HipPrefillPlan(projection, attention)


__all__ = ["HipPrefillPlan", "hip_prefill_plan", "PROJECTION_LABELS", "ATTENTION_KINDS", "ExpMode"]
