"""HIP graph capture of the C-ABI entry points (through torch.cuda.graph).

The entry points launch only kernels on the caller's stream (no allocation,
memset or host synchronisation), so a graph replays them exactly.  Each test
captures a call sequence, replays the graph several times with eager work and
synchronisations between the replays, and compares every replay bit for bit
with the same sequence run eagerly: the kernels and their reduction orders are
deterministic, so the results must be identical.
"""

import pytest
import torch

from lrnnx_amd import causal_conv1d_fn, layer_norm_fn, selective_scan_cuda, selective_state_update

pytestmark = pytest.mark.gpu

REPLAYS = 4


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = fn()
    return g, outs


def _eager_noise(dev):
    a = torch.randn(256, 256, device=dev)
    (a @ a).sum().item()
    torch.cuda.synchronize()


def _flat(outs):
    return [t for t in outs if isinstance(t, torch.Tensor)]


def _check_replays(dev, fn, ref):
    g, outs = _capture(fn)
    outs = _flat(outs)
    for k in range(REPLAYS):
        g.replay()
        torch.cuda.synchronize()
        for i, (o, r) in enumerate(zip(outs, ref)):
            assert torch.equal(o, r), f"replay {k}, output {i} differs from the eager result"
        _eager_noise(dev)


def test_graph_selective_scan_fwd_bwd(dev):
    g = torch.Generator(device=dev).manual_seed(31)
    b, d, L, n = 2, 128, 256, 16
    bf = torch.bfloat16
    u = torch.randn(b, d, L, device=dev, generator=g).to(bf)
    delta = (0.5 * torch.randn(b, d, L, device=dev, generator=g)).to(bf)
    z = torch.randn(b, d, L, device=dev, generator=g).to(bf)
    A = -torch.rand(d, n, device=dev, generator=g) - 0.5
    B = torch.randn(b, 1, n, L, device=dev, generator=g).to(bf)
    C = torch.randn(b, 1, n, L, device=dev, generator=g).to(bf)
    Dv = torch.randn(d, device=dev, generator=g)
    db = 0.1 * torch.randn(d, device=dev, generator=g)
    dout = torch.randn(b, d, L, device=dev, generator=g).to(bf)

    def fn():
        out, x, out_z = selective_scan_cuda.fwd(u, delta, A, B, C, Dv, z, db, None, True, "mamba")
        grads = selective_scan_cuda.bwd(u, delta, A, B, C, Dv, z, db, None, dout, x, out, None, True, False,
                                        "mamba")
        return [out, x, out_z] + list(grads)

    ref = [t.clone() for t in _flat(fn())]
    torch.cuda.synchronize()
    _check_replays(dev, fn, ref)


def test_graph_layer_norm_and_conv(dev):
    g = torch.Generator(device=dev).manual_seed(32)
    bf = torch.bfloat16
    x = torch.randn(4, 64, 512, device=dev, generator=g).to(bf).requires_grad_()
    res = torch.randn(4, 64, 512, device=dev, generator=g).requires_grad_()
    w = (1 + 0.1 * torch.randn(512, device=dev, generator=g)).requires_grad_()
    dy = torch.randn(4, 64, 512, device=dev, generator=g).to(bf)
    dres = torch.randn(4, 64, 512, device=dev, generator=g)
    xc = torch.randn(2, 256, 1000, device=dev, generator=g).to(bf).requires_grad_()
    cw = (0.5 * torch.randn(256, 4, device=dev, generator=g)).requires_grad_()
    cb = (0.1 * torch.randn(256, device=dev, generator=g)).requires_grad_()
    dco = torch.randn(2, 256, 1000, device=dev, generator=g).to(bf)

    def fn():
        y, ro = layer_norm_fn(x, w, None, residual=res, prenorm=True, residual_in_fp32=True, eps=1e-5,
                              is_rms_norm=True)
        gx, gr, gw = torch.autograd.grad([y, ro], [x, res, w], [dy, dres])
        co = causal_conv1d_fn(xc, cw, cb, activation="silu")
        gxc, gcw, gcb = torch.autograd.grad(co, [xc, cw, cb], dco)
        return [y.detach(), ro.detach(), gx, gr, gw, co.detach(), gxc, gcw, gcb]

    ref = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    _check_replays(dev, fn, ref)


def test_graph_decode_step_updates_state_in_place(dev):
    """A 3-layer decode step (the graph-captured step of generation): every
    replay advances the states exactly as the eager step does."""
    g = torch.Generator(device=dev).manual_seed(33)
    bf = torch.bfloat16
    Bt, D, N = 8, 256, 16
    layers = []
    for _ in range(3):
        layers.append(dict(
            state=(0.1 * torch.randn(Bt, D, N, device=dev, generator=g)).to(bf),
            x=torch.randn(Bt, D, device=dev, generator=g).to(bf),
            dt=torch.randn(Bt, D, device=dev, generator=g).to(bf),
            A=-torch.rand(D, N, device=dev, generator=g) - 0.5,
            B=torch.randn(Bt, N, device=dev, generator=g).to(bf),
            C=torch.randn(Bt, N, device=dev, generator=g).to(bf),
            D=torch.ones(D, device=dev),
            z=torch.randn(Bt, D, device=dev, generator=g).to(bf),
            dt_bias=0.1 * torch.randn(D, device=dev, generator=g)))
    s0 = [p["state"].clone() for p in layers]

    def step():
        return [selective_state_update(p["state"], p["x"], p["dt"], p["A"], p["B"], p["C"], D=p["D"], z=p["z"],
                                       dt_bias=p["dt_bias"], dt_softplus=True) for p in layers]

    # eager reference: REPLAYS consecutive steps from s0
    ref_outs, ref_states = [], []
    for k in range(REPLAYS):
        ref_outs.append([o.clone() for o in step()])
        ref_states.append([p["state"].clone() for p in layers])
    torch.cuda.synchronize()
    graph, outs = _capture(step)
    for p, s in zip(layers, s0):   # warm-up ran the step; restart from s0
        p["state"].copy_(s)
    torch.cuda.synchronize()
    for k in range(REPLAYS):
        graph.replay()
        torch.cuda.synchronize()
        for i, p in enumerate(layers):
            assert torch.equal(outs[i], ref_outs[k][i]), f"step {k}, layer {i}: out differs"
            assert torch.equal(p["state"], ref_states[k][i]), f"step {k}, layer {i}: state differs"
        _eager_noise(dev)
