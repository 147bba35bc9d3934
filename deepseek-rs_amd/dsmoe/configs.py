"""The synthetic layer configurations the benchmark and the parity tests run.

C1  small : d=2048, E=64, I=1408 (zero-padded to 1536: Q2_K and Q8_K need
            multiples of 256), top-6, reference routing (scale 1.5), Q8_0
            shared expert (I_s = 1408), f32 activations.
C2  full  : d=7168, E=256 in 8 groups (top-4 groups), top-8, scale 2.5,
            I=2048, Q8_0 shared expert I_s=2048, bf16-valued activations, T=1.
C3        : C2 with T=32.
C4        : C2 with T=128 (N(0,0.02) router); C4-tie: identical router rows,
            so every logit ties and selection is decided by the bias and
            the lower-index rule.
C5        : C2 with T=2048 and a Zipf(1.1) popularity prior over a seeded
            expert permutation, entered through the selection bias
            (bias += -1.1 ln rank, i.e. in score space after sqrt(softplus)).
C5LOGIT   : C2 with T=2048 and the same prior added to the router logits
            themselves: router column 0 holds f16(-1.1 ln rank) and every
            token's x[0] is 1.0, so logit_e = prior_e + sum_{i>0} W[e,i] x_i
            (the prior enters the reference's own logit arithmetic).
REF       : the reference's own layer (engine/src/model.rs:4,15-18,
            session.rs:21): d=4096, E=256, top-6, no groups, scale 1.5, no
            correction bias, I=2048, Q8_0 shared expert I_s=2048.

Weights are N(0, 0.02) quantized by this library's encoders; router weights
N(0, 0.02) in f16; the correction bias N(0, 0.01).
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np

from . import (FMT_F16, FMT_F32, FMT_IQ2_XXS, FMT_Q2_K, FMT_Q8_0, LayerWeights, MoeConfig, synth)

TID_ROUTER, TID_BIAS, TID_GATE, TID_UP, TID_DOWN, TID_SH_GATE, TID_SH_UP, TID_SH_DOWN, TID_X = range(1, 10)


@dataclass
class Case:
    name: str
    cfg: MoeConfig
    T: int
    d_ff_real: int          # I before padding
    d_ff_shared_real: int
    bf16_x: bool = True
    router_tie: bool = False
    zipf: float = 0.0
    zipf_logit: bool = False  # the prior enters the logits (router column 0, x[:, 0] = 1) instead of the bias
    seed: int = 1234


C2_CFG = MoeConfig(d_model=7168, d_ff=2048, n_expert=256, top_k=8, n_group=8, topk_group=4, route_scale=2.5,
                   swiglu_clamp=10.0, has_bias=True, shared_fmt=0, d_ff_shared=2048)

CASES = {
    "c1": Case("c1", MoeConfig(d_model=2048, d_ff=1536, n_expert=64, top_k=6, n_group=1, topk_group=1,
                               route_scale=1.5, swiglu_clamp=10.0, has_bias=True, shared_fmt=0,
                               d_ff_shared=1408), T=1, d_ff_real=1408, d_ff_shared_real=1408, bf16_x=False),
    "c2": Case("c2", C2_CFG, T=1, d_ff_real=2048, d_ff_shared_real=2048),
    "c3": Case("c3", C2_CFG, T=32, d_ff_real=2048, d_ff_shared_real=2048),
    "c4": Case("c4", C2_CFG, T=128, d_ff_real=2048, d_ff_shared_real=2048),
    "c4tie": Case("c4tie", C2_CFG, T=128, d_ff_real=2048, d_ff_shared_real=2048, router_tie=True),
    "c5": Case("c5", C2_CFG, T=2048, d_ff_real=2048, d_ff_shared_real=2048, zipf=1.1),
    "c5logit": Case("c5logit", C2_CFG, T=2048, d_ff_real=2048, d_ff_shared_real=2048, zipf=1.1, zipf_logit=True),
    "ref": Case("ref", MoeConfig(d_model=4096, d_ff=2048, n_expert=256, top_k=6, n_group=1, topk_group=1,
                                 route_scale=1.5, swiglu_clamp=10.0, has_bias=False, shared_fmt=0,
                                 d_ff_shared=2048), T=1, d_ff_real=2048, d_ff_shared_real=2048),
}


def zipf_bias(E, s, seed):
    """-s ln(rank) for a seeded random assignment of ranks 1..E to experts."""
    rng = np.random.default_rng(seed)
    rank = rng.permutation(E) + 1
    return (-s * np.log(rank)).astype(np.float32)


def make_weights(case: Case, layer: int = 0, device="cuda") -> LayerWeights:
    """Generate one layer's quantized weights for `case` (device or 'cpu')."""
    import torch
    c = case.cfg
    base = (case.seed, layer * 16)
    seed, off = base
    E, d, I, Ir = c.n_expert, c.d_model, c.d_ff, case.d_ff_real
    if case.router_tie:
        row = synth(FMT_F16, seed, off + TID_ROUTER, 1, 1, d, sigma=0.02, device=device)
        router = row.reshape(1, d).expand(E, d).contiguous()
    else:
        router = synth(FMT_F16, seed, off + TID_ROUTER, 1, E, d, sigma=0.02, device=device)
    bias = synth(FMT_F32, seed, off + TID_BIAS, 1, 1, E, sigma=0.01, device=device).reshape(E).clone()
    if case.zipf > 0 and case.zipf_logit:
        # logits are sum_i W[e,i] x_i and every token has x[0] = 1 (make_x), so
        # column 0 adds the prior to each expert's logit
        prior = torch.from_numpy(zipf_bias(E, case.zipf, seed)).to(torch.float16)
        router = router.clone()
        router.view(torch.int16).reshape(E, d)[:, 0] = prior.view(torch.int16).to(router.device)
    elif case.zipf > 0:
        bias += torch.from_numpy(zipf_bias(E, case.zipf, seed)).to(bias.device)
    gate = synth(FMT_IQ2_XXS, seed, off + TID_GATE, E, I, d, rows_real=Ir, sigma=0.02, device=device)
    up = synth(FMT_IQ2_XXS, seed, off + TID_UP, E, I, d, rows_real=Ir, sigma=0.02, device=device)
    down = synth(FMT_Q2_K, seed, off + TID_DOWN, E, d, I, cols_real=Ir, sigma=0.02, device=device)
    Is, Isr = c.d_ff_shared, case.d_ff_shared_real
    if c.shared_fmt == 0:
        shg = synth(FMT_Q8_0, seed, off + TID_SH_GATE, 1, Is, d, sigma=0.02, device=device)
        shu = synth(FMT_Q8_0, seed, off + TID_SH_UP, 1, Is, d, sigma=0.02, device=device)
        shd = synth(FMT_Q8_0, seed, off + TID_SH_DOWN, 1, d, Is, sigma=0.02, device=device)
    elif c.shared_fmt == 1:
        shg = synth(FMT_IQ2_XXS, seed, off + TID_SH_GATE, 1, Is, d, rows_real=Isr, sigma=0.02, device=device)
        shu = synth(FMT_IQ2_XXS, seed, off + TID_SH_UP, 1, Is, d, rows_real=Isr, sigma=0.02, device=device)
        shd = synth(FMT_Q2_K, seed, off + TID_SH_DOWN, 1, d, Is, cols_real=Isr, sigma=0.02, device=device)
    else:
        shg = shu = shd = None
    return LayerWeights(router, bias if c.has_bias else None, gate, up, down, shg, shu, shd)


def make_x(case: Case, T: int | None = None, step: int = 0, device="cuda"):
    """Activations [T][d] f32, N(0,1) (rounded to bf16 values for C2-C5)."""
    import torch
    T = case.T if T is None else T
    x = synth(FMT_F32, case.seed, 1000 + step * 16 + TID_X, 1, T, case.cfg.d_model, sigma=1.0, device=device)
    x = x.reshape(T, case.cfg.d_model)
    if case.bf16_x:
        x = x.to(torch.bfloat16).to(torch.float32)
    if case.zipf_logit:
        x[:, 0] = 1.0  # carries the router's prior column (make_weights)
    return x.contiguous()


def with_tokens(case: Case, T: int) -> Case:
    return replace(case, T=T)
