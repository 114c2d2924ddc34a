"""Site routing samplers: which sites take the decomposed output at each position.

Mirrors `param_decomp/param_decomp/core/recon.py:214-265` (`UniformKRouting`,
`StaticProbabilityRouting`, `AllRouting`, `routing_sampler_from_config`). A sampler is
called with a key and the leading shape and returns `{site: bool[*leading_shape]}` (or
None for AllRouting), drawn on the GPU by `pd_route_uniform_k` / `pd_route_static_p`.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from param_decomp_amd import _lib as L
from param_decomp_amd import ops
from param_decomp_amd.prng import Key

Routes = dict[str, torch.Tensor] | None


def _split_routes(routes: torch.Tensor, sites: tuple[str, ...], leading_shape) -> dict[str, torch.Tensor]:
    flat = routes.view(torch.bool)
    return {name: flat[j].reshape(tuple(leading_shape)) for j, name in enumerate(sites)}


@dataclass(frozen=True)
class UniformKRouting:
    """A uniform nonempty subset of sites, independently at each position
    (`core/recon.py:218-231`)."""

    sites: tuple[str, ...]
    device: str | torch.device = "cuda"
    layout: int = L.LAYOUT_PARTITIONABLE

    def __call__(self, key: Key, leading_shape) -> Routes:
        n = int(math.prod(leading_shape))
        routes = ops.route_uniform_k(key, len(self.sites), n, self.device, self.layout)
        return _split_routes(routes, self.sites, leading_shape)


@dataclass(frozen=True)
class StaticProbabilityRouting:
    """Each site routed independently with probability p (`core/recon.py:233-244`)."""

    sites: tuple[str, ...]
    p: float
    device: str | torch.device = "cuda"
    layout: int = L.LAYOUT_PARTITIONABLE

    def __call__(self, key: Key, leading_shape) -> Routes:
        n = int(math.prod(leading_shape))
        routes = ops.route_static_p(key, len(self.sites), self.p, n, self.device, self.layout)
        return _split_routes(routes, self.sites, leading_shape)


@dataclass(frozen=True)
class AllRouting:
    """Every position routed to every site (`core/recon.py:247-252`)."""

    def __call__(self, key: Key, leading_shape) -> Routes:
        return None


def routing_sampler_from_config(routing: dict, sites: tuple[str, ...], device="cuda"):
    """`core/recon.py:255-265` over the config's `type` tag: "uniform_k_subset",
    "static_probability" (with `p`) or "all"."""
    kind = routing.get("type", "uniform_k_subset")
    if kind == "uniform_k_subset":
        return UniformKRouting(tuple(sites), device)
    if kind == "static_probability":
        return StaticProbabilityRouting(tuple(sites), float(routing["p"]), device)
    if kind == "all":
        return AllRouting()
    raise ValueError(f"unknown routing type {kind!r}")
