"""The allocation-free masked-linear backward (`pd_masked_linear_bwd_noalloc`) against
`pd_masked_linear_bwd` through the C ABI: two calls in a row, the second with a smaller
input, each bit-identical to the workspace entry point on the same inputs (the two share
their kernels); requests above the fixed scratch size are refused on the host."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(rng, T, d_in, d_out, C, device, dtype):
    def t(*shape, scale=1.0):
        return torch.tensor(rng.normal(size=shape) * scale, dtype=torch.float32, device=device).to(dtype)

    x, V, U, W = t(T, d_in), t(d_in, C, scale=d_in**-0.5), t(C, d_out, scale=C**-0.5), t(d_out, d_in, scale=0.1)
    mask = torch.tensor(rng.uniform(size=(T, C)), dtype=torch.float32, device=device).to(dtype)
    delta = torch.tensor(rng.uniform(size=T), dtype=torch.float32, device=device).to(dtype)
    route = torch.tensor(rng.uniform(size=T) > 0.25, dtype=torch.uint8, device=device)
    g = t(T, d_out)
    return x, V, U, W, mask, delta, route, g


def _backward(L, entry, dtype, T, d_in, d_out, C, x, V, U, W, mask, delta, route, g):
    dev = x.device
    code = L.dtype_code(dtype)
    xV = torch.empty(T, C, dtype=dtype, device=dev)
    acts = torch.empty(T, C, dtype=dtype, device=dev)
    out = torch.empty(T, d_out, dtype=dtype, device=dev)
    L.call("pd_masked_linear_fwd", code, T, d_in, d_out, C, L.ptr(x), L.ptr(V), L.ptr(U), L.ptr(W), L.ptr(mask),
           L.ptr(delta), L.ptr(route), L.ptr(out), L.ptr(xV), L.ptr(acts), L.stream())
    grads = [torch.full(shape, float("nan"), dtype=dtype, device=dev)
             for shape in ((T, d_in), (d_in, C), (C, d_out), (T, C), (T,))]
    args = [code, T, d_in, d_out, C, L.ptr(x), L.ptr(V), L.ptr(U), L.ptr(W), L.ptr(mask), L.ptr(delta), L.ptr(route),
            L.ptr(xV), L.ptr(acts), L.ptr(g)] + [L.ptr(t) for t in grads]
    if entry == "pd_masked_linear_bwd":
        ws = L.workspace(L.load().pd_masked_linear_bwd_workspace_size(code, T, d_out, C), dev)
        L.call(entry, *args, L.ptr(ws), ws.numel(), L.stream())
    else:
        L.call(entry, *args, L.stream())
    torch.cuda.synchronize()
    return grads


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_backward_matches_the_workspace_entry_point(device, dtype):
    from param_decomp_amd import _lib as L

    rng = np.random.default_rng(41)
    # a large call, then a smaller one: the second reuses the region the first filled
    for T, d_in, d_out, C in ((2048, 256, 768, 4096), (200, 64, 136, 96)):
        inp = _inputs(rng, T, d_in, d_out, C, device, dtype)
        want = _backward(L, "pd_masked_linear_bwd", dtype, T, d_in, d_out, C, *inp)
        got = _backward(L, "pd_masked_linear_bwd_noalloc", dtype, T, d_in, d_out, C, *inp)
        for name, a, b in zip(("dx", "dV", "dU", "dmask", "d_delta"), got, want):
            assert torch.isfinite(b.float()).all(), name
            assert torch.equal(a, b), f"{name} differs at T={T}"


def test_noalloc_backward_refuses_requests_above_its_scratch(device):
    from param_decomp_amd import _lib as L

    limit = 64 << 20
    T, C, d_out = 8192, 4096, 1024  # bf16: 2*T*C + 2*T*d_out + 512 bytes > 64 MiB
    assert L.load().pd_masked_linear_bwd_workspace_size(L.BF16, T, d_out, C) > limit
    dummy = torch.zeros(16, dtype=torch.bfloat16, device=device)
    p = L.ptr(dummy)
    with pytest.raises(L.PDError, match="above the fixed"):
        L.call("pd_masked_linear_bwd_noalloc", L.BF16, T, 64, d_out, C, p, p, p, p, p, None, None, p, p, p, p, p, p,
               None, None, L.stream())


def test_noalloc_backward_replays_under_graph_capture(device):
    """Captured into a HIP graph (torch.cuda.graph) after one eager call on the device, the
    allocation-free backward replays with new inputs written into the captured buffers;
    every replay, with eager calls of the workspace entry point between them, is
    bit-identical to pd_masked_linear_bwd on the same inputs."""
    from param_decomp_amd import _lib as L

    dtype, T, d_in, d_out, C = torch.bfloat16, 512, 256, 384, 1024
    code = L.dtype_code(dtype)
    rng = np.random.default_rng(7)
    static = [t.clone() for t in _inputs(rng, T, d_in, d_out, C, device, dtype)]
    x, V, U, W, mask, delta, route, g = static
    xV = torch.empty(T, C, dtype=dtype, device=device)
    acts = torch.empty(T, C, dtype=dtype, device=device)
    out = torch.empty(T, d_out, dtype=dtype, device=device)
    grads = [torch.zeros(shape, dtype=dtype, device=device) for shape in ((T, d_in), (d_in, C), (C, d_out), (T, C), (T,))]

    def forward():
        L.call("pd_masked_linear_fwd", code, T, d_in, d_out, C, L.ptr(x), L.ptr(V), L.ptr(U), L.ptr(W), L.ptr(mask),
               L.ptr(delta), L.ptr(route), L.ptr(out), L.ptr(xV), L.ptr(acts), L.stream())

    def noalloc():
        L.call("pd_masked_linear_bwd_noalloc", code, T, d_in, d_out, C, L.ptr(x), L.ptr(V), L.ptr(U), L.ptr(W),
               L.ptr(mask), L.ptr(delta), L.ptr(route), L.ptr(xV), L.ptr(acts), L.ptr(g),
               *[L.ptr(t) for t in grads], L.stream())

    forward()
    noalloc()  # the eager call that looks the scratch region up on this device
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=device)  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        noalloc()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        noalloc()
    torch.cuda.synchronize()
    for replay in range(3):
        for dst, src in zip(static, _inputs(rng, T, d_in, d_out, C, device, dtype)):
            dst.copy_(src)
        forward()
        for t in grads:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in grads]
        want = _backward(L, "pd_masked_linear_bwd", dtype, T, d_in, d_out, C, *static)
        for name, a, b in zip(("dx", "dV", "dU", "dmask", "d_delta"), got, want):
            assert torch.isfinite(b.float()).all(), name
            assert torch.equal(a, b), f"{name} differs on replay {replay}"
