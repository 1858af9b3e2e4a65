"""The benchmark configurations (synthetic, seeded) and their small tensors.

Config 0..3 share one layer of weights (seed 0xC0, layer 0): the router, the
norm weight and all 193 experts. Each config has its own input seed. Config 3
replaces the expert bias with the Zipf-like skew. Config 4 stacks 79 layers
(seed 0xC4, layer l) and decodes one token.

Distributions (hy3 MoE layer):
  x       ~ N(0, 1)            [T x 4096]  kind T_X,      seed = config seed
  norm_w  ~ 1 + N(0, 0.02)     [4096]      kind T_NORM,   weight seed
  router  ~ N(0, 0.02)         [192x4096]  kind T_ROUTER, weight seed
  bias    ~ U(-0.1, 0.1)       [192]       kind T_BIAS,   weight seed
          or 0.5*(1/(rank+1))^0.8 over a seeded permutation (config 3)
  experts ~ N(0, 0.02) -> Q4_K kinds T_GATE/T_UP/T_DOWN, expert index 192 =
          shared expert (generated on the device, hy3x_synth_layer_experts).
"""
from dataclasses import dataclass

import numpy as np

from . import (D_MODEL, N_EXPERT, T_BIAS, T_NORM, T_ROUTER, T_X, synth_key, synth_normal,
               synth_uniform_sym, synth_zipf_bias)

WEIGHT_SEED = 0xC0


@dataclass(frozen=True)
class Config:
    index: int
    name: str
    T: int
    input_seed: int
    weight_seed: int = WEIGHT_SEED
    zipf_bias: bool = False
    n_layers: int = 1
    K: int = 8


CONFIGS = [
    Config(0, "decode_b1", 1, 0xC0),
    Config(1, "decode_b32", 32, 0xC1),
    Config(2, "prefill_512", 512, 0xC2),
    Config(3, "prefill_4096_zipf", 4096, 0xC3, zipf_bias=True),
    Config(4, "stack79_decode_b1", 1, 0xC4, weight_seed=0xC4, n_layers=79),
]


def layer_small_tensors(weight_seed, layer=0, zipf=False, zipf_seed=None):
    """norm_w, router, bias (host fp32) of one synthetic layer."""
    norm_w = synth_normal(D_MODEL, synth_key(weight_seed, layer, T_NORM), 0.02, 1.0)
    router = synth_normal(N_EXPERT * D_MODEL, synth_key(weight_seed, layer, T_ROUTER), 0.02)
    if zipf:
        bias = synth_zipf_bias(N_EXPERT, weight_seed if zipf_seed is None else zipf_seed)
    else:
        bias = synth_uniform_sym(N_EXPERT, synth_key(weight_seed, layer, T_BIAS), 0.1)
    return norm_w, router.reshape(N_EXPERT, D_MODEL), bias


def inputs(input_seed, T, first_token=0):
    """x[T x 4096] for tokens first_token .. first_token+T-1."""
    x = synth_normal(T * D_MODEL, synth_key(input_seed, 0, T_X), 1.0, 0.0,
                     first=first_token * D_MODEL)
    return x.reshape(T, D_MODEL)


def config_tensors(cfg, layer=0):
    zipf_seed = cfg.input_seed if cfg.zipf_bias else None
    return layer_small_tensors(cfg.weight_seed, layer, cfg.zipf_bias, zipf_seed)


def expert_bytes(n_unique):
    return n_unique * 10616832


def algorithmic_bytes(T, n_unique_incl_shared):
    """Bytes one forward must move at minimum (weights once, x in, y out)."""
    return (n_unique_incl_shared * 10616832 + 192 * 4096 * 4 + 4096 * 4 + 192 * 4
            + T * 4096 * 4 * 2)


def algorithmic_flops(T, K):
    return T * ((K + 1) * 2 * 3 * 1536 * 4096 + 2 * 192 * 4096)


def unique_experts(ids):
    return int(np.unique(np.asarray(ids).ravel()).size) + 1
