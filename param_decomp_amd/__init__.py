"""MI355X-native (gfx950) masked-component hot path of goodfire-ai/param-decomp.

Host API mirrors the reference's seams (`decomposed_linear.site_forward`, `masking`,
`squashing`, `losses`, `routed.experts.grouped_matmul` with backend "hip"); all
arithmetic runs in the HIP library `_lib/libpd_mi355x.so` through its C ABI
(`include/pd_mi355x.h`).
"""

__all__ = ["build", "ops", "prng"]


def build(verbose: bool = False) -> str:
    from param_decomp_amd import builder as _b

    return _b.build(verbose=verbose)
