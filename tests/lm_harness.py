"""Config-4 harness: a Mamba language model built from this package's
kernels (RMSNorm with the fused residual add, causal conv1d and its decode
update, the selective scan and the one-step state update) plus torch GEMMs,
random-initialised.  Test / benchmark infrastructure: lrnnx's model code is
out of scope for the package, so this mirrors just enough of it to drive the
hot path the way the reference's models do.

Mirrors (reference files):
  MambaMixer.__init__ / forward / step / allocate_inference_cache
      lrnnx/models/ltv/mamba.py:66-178, :179-353 (the selective_scan_fn path
      with causal_conv1d_fn), :355-496 (selective_state_update path),
      :498-548
  Block (fused add + RMSNorm, prenorm)   lrnnx/layers/block.py:17-118
  MambaLM.forward / step                 lrnnx/architectures/language_model.py:
      344-452 (LRNNModel.step), :454-510 (LRNNModel.forward), :653-727
      (LRNNLMHeadModel.step / forward), tied embeddings, vocab padded to a
      multiple of 8 (:563-567), _init_weights (:156-195)
  capture_decode / greedy_decode         lrnnx/utils/generation.py:74-174 (warm-up
      on a side stream, capture of one step, replay)

Differences, both deliberate: the reference's LM prefill never fills the
Mamba caches (block.py:90-98 retries the mixer without ``inference_params``);
``forward(..., caches=...)`` here fills them, as Mamba.forward does when
called with ``inference_cache``, so that decoding can continue from a
prefill.  The captured decode step also feeds its greedy token back into its
input buffer, so replays need no host work between tokens.
"""

from __future__ import annotations

import math
from collections import namedtuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from lrnnx_amd import (RMSNorm, causal_conv1d_fn, causal_conv1d_update, layer_norm_fn, selective_scan_fn,
                       selective_state_update)

CausalLMOutput = namedtuple("CausalLMOutput", ["logits"])


class MambaMixer(nn.Module):
    def __init__(self, d_model, d_state=16, d_conv=4, expand=2, dt_min=0.001, dt_max=0.1, dt_init_floor=1e-4,
                 device=None, dtype=None):
        super().__init__()
        fk = {"device": device, "dtype": dtype}
        self.d_model, self.d_state, self.d_conv = d_model, d_state, d_conv
        self.d_inner = expand * d_model
        self.dt_rank = math.ceil(d_model / 16)
        self.in_proj = nn.Linear(d_model, 2 * self.d_inner, bias=False, **fk)
        self.conv1d = nn.Conv1d(self.d_inner, self.d_inner, d_conv, groups=self.d_inner, padding=d_conv - 1,
                                bias=True, **fk)
        self.x_proj = nn.Linear(self.d_inner, self.dt_rank + 2 * d_state, bias=False, **fk)
        self.dt_proj = nn.Linear(self.dt_rank, self.d_inner, bias=True, **fk)
        std = self.dt_rank ** -0.5
        nn.init.uniform_(self.dt_proj.weight, -std, std)
        dt = torch.exp(torch.rand(self.d_inner, device=device) * (math.log(dt_max) - math.log(dt_min))
                       + math.log(dt_min)).clamp(min=dt_init_floor)
        with torch.no_grad():
            self.dt_proj.bias.copy_(dt + torch.log(-torch.expm1(-dt)))   # inverse softplus
        self.dt_proj.bias._no_reinit = True
        A = torch.arange(1, d_state + 1, dtype=torch.float32, device=device).repeat(self.d_inner, 1)
        self.A_log = nn.Parameter(torch.log(A))                          # fp32
        self.D = nn.Parameter(torch.ones(self.d_inner, device=device))   # fp32
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=False, **fk)

    def allocate_inference_cache(self, batch_size, dtype=None):
        dev = self.out_proj.weight.device
        return {"conv_state": torch.zeros(batch_size, self.d_inner, self.d_conv, device=dev,
                                          dtype=dtype or self.conv1d.weight.dtype),
                "lrnn_state": torch.zeros(batch_size, self.d_inner, self.d_state, device=dev,
                                          dtype=dtype or self.dt_proj.weight.dtype),
                "seqlen_offset": 0}

    def forward(self, hidden_states, cache=None):
        b, L, _ = hidden_states.shape
        # (b, 2 d_inner, L) in one GEMM; x and z are strided halves of it
        xz = (self.in_proj.weight @ hidden_states.reshape(b * L, -1).t()).reshape(-1, b, L).transpose(0, 1)
        A = -torch.exp(self.A_log.float())
        x, z = xz.chunk(2, dim=1)
        if cache is not None:
            cache["conv_state"].copy_(F.pad(x, (self.d_conv - L, 0)))
        x = causal_conv1d_fn(x, self.conv1d.weight.squeeze(1), self.conv1d.bias, activation="silu")
        x_dbl = self.x_proj(x.transpose(1, 2).reshape(b * L, -1))
        dt, Bm, Cm = torch.split(x_dbl, [self.dt_rank, self.d_state, self.d_state], dim=-1)
        Bm = Bm.reshape(b, L, -1).transpose(1, 2).contiguous()
        Cm = Cm.reshape(b, L, -1).transpose(1, 2).contiguous()
        dt = (self.dt_proj.weight @ dt.t()).reshape(-1, b, L).transpose(0, 1)
        y = selective_scan_fn(x, dt, A, Bm, Cm, self.D.float(), z=z, delta_bias=self.dt_proj.bias.float(),
                              delta_softplus=True, return_last_state=cache is not None)
        if cache is not None:
            y, last_state = y
            cache["lrnn_state"].copy_(last_state)
            cache["seqlen_offset"] = L
        return self.out_proj(y.transpose(1, 2))

    def step(self, hidden_states, cache):
        xz = self.in_proj(hidden_states.squeeze(1))
        x, z = xz.chunk(2, dim=-1)
        x = causal_conv1d_update(x, cache["conv_state"], self.conv1d.weight.squeeze(1), self.conv1d.bias, "silu")
        x_db = self.x_proj(x)
        dt = F.linear(x_db[:, :self.dt_rank], self.dt_proj.weight)
        Bm = x_db[:, self.dt_rank:self.dt_rank + self.d_state]
        Cm = x_db[:, -self.d_state:]
        A = -torch.exp(self.A_log.float())
        y = selective_state_update(cache["lrnn_state"], x, dt, A, Bm, Cm, self.D, z=z, dt_bias=self.dt_proj.bias,
                                   dt_softplus=True)
        cache["seqlen_offset"] += 1
        return self.out_proj(y).unsqueeze(1)


class Block(nn.Module):
    def __init__(self, d_model, d_state, eps, device=None, dtype=None):
        super().__init__()
        self.norm = RMSNorm(d_model, eps=eps, device=device, dtype=dtype)
        self.mixer = MambaMixer(d_model, d_state, device=device, dtype=dtype)

    def forward(self, hidden_states, residual=None, cache=None):
        hidden_states, residual = layer_norm_fn(hidden_states, self.norm.weight, None, residual=residual,
                                                prenorm=True, eps=self.norm.eps, is_rms_norm=True)
        return self.mixer(hidden_states, cache), residual


def _init_weights(module, n_layer, initializer_range=0.02):
    if isinstance(module, nn.Linear):
        if module.bias is not None and not getattr(module.bias, "_no_reinit", False):
            nn.init.zeros_(module.bias)
    elif isinstance(module, nn.Embedding):
        nn.init.normal_(module.weight, std=initializer_range)
    for name, p in module.named_parameters():
        if name == "out_proj.weight":
            nn.init.kaiming_uniform_(p, a=math.sqrt(5))
            with torch.no_grad():
                p /= math.sqrt(n_layer)


class MambaLM(nn.Module):
    """LRNNLMHeadModel(d_model, d_state, n_layer, vocab_size, mixer_types=["Mamba"] * n_layer) with the
    reference's defaults: RMSNorm, fused add + norm, no MLP, tied embeddings."""

    def __init__(self, d_model=768, d_state=16, n_layer=24, vocab_size=50280, eps=1e-5, device=None, dtype=None):
        super().__init__()
        fk = {"device": device, "dtype": dtype}
        vocab = vocab_size + (-vocab_size % 8)
        self.embedding = nn.Embedding(vocab, d_model, **fk)
        self.layers = nn.ModuleList([Block(d_model, d_state, eps, **fk) for _ in range(n_layer)])
        self.norm_f = RMSNorm(d_model, eps=eps, **fk)
        self.lm_head = nn.Linear(d_model, vocab, bias=False, **fk)
        self.apply(lambda m: _init_weights(m, n_layer))
        self.lm_head.weight = self.embedding.weight

    def allocate_inference_cache(self, batch_size):
        return {i: layer.mixer.allocate_inference_cache(batch_size) for i, layer in enumerate(self.layers)}

    def _head(self, hidden_states, residual):
        h = layer_norm_fn(hidden_states, self.norm_f.weight, None, residual=residual, prenorm=False,
                          eps=self.norm_f.eps, is_rms_norm=True)
        return self.lm_head(h)

    def forward(self, input_ids, caches=None, num_last_tokens=0):
        h = self.embedding(input_ids)
        residual = None
        for i, layer in enumerate(self.layers):
            h, residual = layer(h, residual, None if caches is None else caches[i])
        if num_last_tokens > 0:
            h, residual = h[:, -num_last_tokens:], residual[:, -num_last_tokens:]
        return CausalLMOutput(logits=self._head(h, residual))

    def step(self, input_ids, caches):
        h = self.embedding(input_ids)
        residual = None
        for i, layer in enumerate(self.layers):
            normed, residual = layer_norm_fn(h, layer.norm.weight, None, residual=residual, prenorm=True,
                                             eps=layer.norm.eps, is_rms_norm=True)
            h = layer.mixer.step(normed, caches[i])
        return CausalLMOutput(logits=self._head(h, residual))


class DecodeGraph:
    """One greedy decode step of ``model`` captured as a HIP graph
    (generation.py:74-174's pattern): static token buffer (b, 1), caches of
    the model, logits of the step; the step writes its argmax token back to
    the input buffer, so ``replay()`` n times decodes n tokens."""

    def __init__(self, model, batch_size, n_warmups=3, argmax_in_graph=True):
        dev = model.embedding.weight.device
        self.model = model
        self.caches = model.allocate_inference_cache(batch_size)
        self.ids = torch.zeros(batch_size, 1, dtype=torch.long, device=dev)
        self.argmax_in_graph = argmax_in_graph

        def step():
            logits = model.step(self.ids, self.caches).logits
            if argmax_in_graph:
                self.ids.copy_(logits[:, -1].argmax(-1, keepdim=True))
            return logits

        self._step = step
        s = torch.cuda.Stream(device=dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s), torch.no_grad():
            for _ in range(n_warmups):
                step()
        torch.cuda.current_stream(dev).wait_stream(s)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.no_grad():
            self.logits = step()

    def reset(self, ids=None):
        """Zero the caches (a fill kernel each; no memset node is recorded)
        and set the input token."""
        for c in self.caches.values():
            c["conv_state"].zero_()
            c["lrnn_state"].zero_()
        if ids is not None:
            self.ids.copy_(ids)

    def replay(self):
        self.graph.replay()
        if not self.argmax_in_graph:
            self.ids.copy_(self.logits[:, -1].argmax(-1, keepdim=True))
        return self.logits


def build(dtype=torch.bfloat16, device="cuda", seed=0, **kw):
    torch.manual_seed(seed)
    return MambaLM(device=device, dtype=dtype, **kw).eval()
