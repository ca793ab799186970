"""vagus_amd — the gated delta-rule linear-attention core (GDN / KDA) on
MI355X (gfx950): hand-written HIP kernels behind a C ABI (include/vagus_gdr.h),
called from Python with the reference's operator signatures.

    from vagus_amd import chunk_gated_delta_rule, chunk_kda, fused_recurrent_gated_delta_rule
"""
from .ops import (chunk_gated_delta_rule, chunk_kda, chunk_simple_gla,  # noqa: F401
                  fused_recurrent_gated_delta_rule, fused_recurrent_kda, hip_recurrent, hip_scan)

__all__ = ['chunk_gated_delta_rule', 'chunk_kda', 'chunk_simple_gla',
           'fused_recurrent_gated_delta_rule', 'fused_recurrent_kda', 'hip_scan', 'hip_recurrent']
