"""Shared assertion for the MoE step's expert selection against the MoE oracle."""

import numpy as np

from oracle import moe_oracle as mo


def assert_routing_matches(got, ref, layer, k, max_frac=0.01):
    """The GPU's expert selection equals the oracle's own (bit-exact) on all but at most
    `max_frac` of the tokens, and every token that differs is a near-tie: its selection
    is the top-k of logits within one bf16 ulp of the oracle's. The bf16 router products
    of two correct fp32-accumulating implementations can round to adjacent values; the
    oracle is then run on the GPU's selection so that every value downstream is
    compared on the same routing. The tie-break itself is checked bit-exact on given
    logits by the router top-k test."""
    own = ref["own_top_idx"][layer]
    bad = np.nonzero((got != own).any(axis=1))[0]
    assert len(bad) <= max(1, int(max_frac * len(got))), f"layer {layer}: {len(bad)} tokens route differently"
    for t in bad:
        assert mo.selection_within_ulps(ref["logits_raw"][layer][t], got[t], k), (
            f"layer {layer} token {t}: {got[t]} vs oracle {own[t]} is not a near-tie")
