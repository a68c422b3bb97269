"""AB-Attention for MI355X (gfx950): IBCS selection, SIP sampling and the
weighted paged prefill behind the reference's Q/K/V API."""
from .attention import SamplePlan, ab_attention, apply_plan, build_plan

__all__ = ["SamplePlan", "ab_attention", "apply_plan", "build_plan"]
