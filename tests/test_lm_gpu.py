"""Config 4 on the GPU: the 24-layer Mamba language model of tests/lm_harness.py
(d_model 768, d_state 16, vocab 50280; the reference's LRNNLMHeadModel with
mixer "Mamba") run on this package's kernels.

* Step == forward, the reference's parallel == recurrent bar
  (tests/models/test_ltv/test_mamba.py:51-87), at the LM level and in fp32:
  a prefill that fills the caches, then the last k prompt tokens decoded one
  by one, reproduce the full forward's last-k logits; decoding from zero
  caches reproduces the forward's first logits.  Tolerance rtol 1e-3,
  atol 1e-4 (the reference test uses 3e-3 / 5e-3).
* The graph-captured greedy decode step at config 4's batch (64, bf16):
  every replay matches an eager step sequence fed the same tokens.
* The decode update at config 4's shape (64 x 1536 x 16, bf16 state) against
  the oracle.
"""

import pytest
import torch

from lrnnx_amd import selective_state_update
from oracle import scan_ref as R
from tests import lm_harness as H
from tests.parity import close

pytestmark = pytest.mark.gpu

VOCAB = 50280


@pytest.fixture(scope="module")
def model_f32(dev):
    return H.build(torch.float32, dev, seed=0)


def test_lm_prefill_then_decode_matches_forward_fp32(dev, model_f32):
    g = torch.Generator(device=dev).manual_seed(1)
    B, T, k = 2, 96, 16
    ids = torch.randint(0, VOCAB, (B, T), generator=g, device=dev)
    with torch.no_grad():
        full = model_f32(ids).logits
        caches = model_f32.allocate_inference_cache(B)
        pre = model_f32(ids[:, :T - k], caches=caches).logits
        steps = [model_f32.step(ids[:, t:t + 1], caches).logits for t in range(T - k, T)]
    torch.cuda.synchronize()
    ref = full.double().cpu()
    close("prefill logits", pre, ref[:, :T - k], 1e-3, 0.0, 1e-4)
    close("decoded last-k logits", torch.cat(steps, 1), ref[:, T - k:], 1e-3, 0.0, 1e-4)


def test_lm_decode_from_zero_matches_forward_fp32(dev, model_f32):
    g = torch.Generator(device=dev).manual_seed(2)
    B, T = 3, 24
    ids = torch.randint(0, VOCAB, (B, T), generator=g, device=dev)
    with torch.no_grad():
        full = model_f32(ids).logits
        caches = model_f32.allocate_inference_cache(B)
        steps = [model_f32.step(ids[:, t:t + 1], caches).logits for t in range(T)]
    torch.cuda.synchronize()
    close("step logits from zero caches", torch.cat(steps, 1), full.double().cpu(), 1e-3, 0.0, 1e-4)


def test_lm_graph_decode_matches_eager_bf16(dev):
    """Replays of the captured greedy step (argmax fed back inside the graph)
    against the same steps run eagerly, compared replay by replay; the
    caches are cleared by fill kernels between the two runs."""
    model = H.build(torch.bfloat16, dev, seed=3)
    B, n = 64, 8
    g = torch.Generator(device=dev).manual_seed(4)
    first = torch.randint(0, VOCAB, (B, 1), generator=g, device=dev)
    dg = H.DecodeGraph(model, B)
    dg.reset(first)
    got_logits, got_ids = [], []
    for _ in range(n):
        got_logits.append(dg.replay().clone())
        got_ids.append(dg.ids.clone())
    torch.cuda.synchronize()
    caches = model.allocate_inference_cache(B)
    ids = first.clone()
    with torch.no_grad():
        for i in range(n):
            logits = model.step(ids, caches).logits
            ids = logits[:, -1].argmax(-1, keepdim=True)
            torch.cuda.synchronize()
            assert torch.isfinite(logits).all()
            assert torch.equal(got_logits[i], logits), f"replay {i}: max diff {(got_logits[i] - logits).abs().max()}"
            assert torch.equal(got_ids[i], ids), f"replay {i}: greedy tokens differ"
    # a second decode from the same start replays identically
    dg.reset(first)
    for i in range(n):
        assert torch.equal(dg.replay(), got_logits[i]), f"second run, replay {i}"


def test_state_update_cfg4_shape(dev):
    """selective_state_update at config 4's decode shape (batch 64, d_inner
    1536, d_state 16, bf16 state, z gate, dt_bias + softplus) against the
    fp64 oracle."""
    g = torch.Generator().manual_seed(7)
    b, d, n = 64, 1536, 16
    bf = torch.bfloat16
    state = (0.1 * torch.randn(b, d, n, generator=g)).to(bf)
    x, dt, z = (torch.randn(b, d, generator=g).to(bf) for _ in range(3))
    A = -torch.arange(1, n + 1, dtype=torch.float32).repeat(d, 1)
    Bm, Cm = torch.randn(b, n, generator=g).to(bf), torch.randn(b, n, generator=g).to(bf)
    D = torch.ones(d)
    dt_bias = 0.1 * torch.randn(d, generator=g)
    st_ref = state.clone().double()
    out_ref = R.selective_state_update_ref(st_ref, x.double(), dt.double(), A.double(), Bm.double(), Cm.double(),
                                           D.double(), z.double(), dt_bias.double(), True, None, "mamba",
                                           compute_dtype=torch.float64)
    st = state.to(dev)
    out = selective_state_update(st, x.to(dev), dt.to(dev), A.to(dev), Bm.to(dev), Cm.to(dev), D.to(dev),
                                 z=z.to(dev), dt_bias=dt_bias.to(dev), dt_softplus=True)
    torch.cuda.synchronize()
    close("state", st, st_ref, 2e-2, 1e-2)
    close("out", out, out_ref, 2e-2, 1e-2)
