"""pom_amd — Polynomial Mixer (PoM) on AMD Instinct MI355X (gfx950).

Drop-in for the reference package ``pom`` (pom/__init__.py:1-2): ``PoM``,
``pom`` and ``PoMRoPE`` keep their signatures; the aggregation, gating and
RoPE steps run in hand-written HIP kernels (libpom_amd.so, C ABI in
include/pom_amd.h).
"""
from .pom import (PoM, pom, pom_activation, polynomial_aggregation_, polynomial_selection_,
                  block_causal)
from .pom_rope import (PoMRoPE, precompute_freqs_1d, precompute_freqs_2d, apply_rope_1d,
                       apply_rope_2d)
from .ops import (poly_agg_mean_hip, poly_agg_masked_hip, poly_agg_causal_hip,
                  poly_agg_block_causal_hip, poly_agg_rope_mean_hip, poly_agg_rope_causal_hip,
                  pom_layer, gate_hip)
from ._lib import available as hip_available

__all__ = ["PoM", "pom", "PoMRoPE", "pom_activation", "polynomial_aggregation_",
           "polynomial_selection_", "block_causal", "precompute_freqs_1d", "precompute_freqs_2d",
           "apply_rope_1d", "apply_rope_2d", "poly_agg_mean_hip", "poly_agg_masked_hip",
           "poly_agg_causal_hip", "poly_agg_block_causal_hip", "poly_agg_rope_mean_hip",
           "poly_agg_rope_causal_hip", "pom_layer", "gate_hip", "hip_available"]
