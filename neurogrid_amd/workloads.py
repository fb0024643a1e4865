"""Measured configurations: shapes, seeded synthetic inputs, algorithmic bytes.

One entry per configuration of the benchmark definition (TinyLlama fp32 on
the CPU path; Mistral-7B fp16 decode and prefill; Llama-2-13B fp16 prefill;
Mistral-Nemo bf16; the int8 quant path at Mistral-7B shapes). Model shapes
follow the reference's presets (pkg/types/config.go) and the models' public
configs. Inputs are drawn with numpy ``Generator(PCG64(seed))`` in the fixed
order listed in each generator, in float32/float64, then rounded to nearest
even into the storage type; "N(0, 4)" and "N(0, 2)" are variances (sigma 2
and sqrt 2).

Algorithmic bytes count each input read once and each output written once
(e = element bytes):
  gather 2 T H e + 4 T        rmsnorm 2 T H e + H e     add+rmsnorm 4 T H e + H e
  swiglu 3 T I e              rope 2 T nh D e + 4 T     residual add 3 T H e
  rmsnorm+int8 T H e + T H + 4 T + H e                  dequant N K + 4 N + 2 N K
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class LayerConfig:
    key: str
    model: str
    dtype: str            # "f16", "bf16" or "f32" (CPU-only)
    T: int                # tokens
    H: int                # hidden
    I: int                # intermediate
    nq: int               # query heads
    nkv: int              # key/value heads
    D: int                # head_dim
    theta: float
    eps: float
    vocab: int
    positions: str        # "arange" or "uniform:<max>"
    ids: str              # "uniform" or "zipf:<s>"
    res_sigma: float = 2.0
    gate_sigma: float = 1.0

    @property
    def e(self) -> int:
        return 4 if self.dtype == "f32" else 2


CONFIGS: dict[str, LayerConfig] = {
    "tinyllama_t1": LayerConfig("tinyllama_t1", "TinyLlama-1.1B", "f32", 1, 2048, 5632, 32, 4, 64, 1e4, 1e-5,
                                32000, "arange", "uniform", 1.0),
    "tinyllama_t128": LayerConfig("tinyllama_t128", "TinyLlama-1.1B", "f32", 128, 2048, 5632, 32, 4, 64, 1e4,
                                  1e-5, 32000, "arange", "uniform", 1.0),
    "mistral7b_decode": LayerConfig("mistral7b_decode", "Mistral-7B", "f16", 64, 4096, 14336, 32, 8, 128, 1e6,
                                    1e-5, 32000, "uniform:4096", "uniform"),
    "mistral7b_prefill": LayerConfig("mistral7b_prefill", "Mistral-7B", "f16", 4096, 4096, 14336, 32, 8, 128, 1e6,
                                     1e-5, 32000, "arange", "uniform"),
    "llama2_13b_prefill": LayerConfig("llama2_13b_prefill", "Llama-2-13B", "f16", 8192, 5120, 13824, 40, 40, 128,
                                      1e4, 1e-5, 32000, "arange", "uniform", 1.0, float(np.sqrt(2.0))),
    "mistral_nemo_bf16": LayerConfig("mistral_nemo_bf16", "Mistral-Nemo-12B", "bf16", 2048, 5120, 14336, 32, 8,
                                     128, 1e6, 1e-5, 131072, "uniform:32768", "zipf:1.1"),
}

QUANT_T, QUANT_H, QUANT_WN, QUANT_WK = 4096, 4096, 14336, 4096


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 -> storage bits (uint16 for 16-bit types, float32 otherwise), RNE."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f16":
        return x.astype(np.float16).view(np.uint16)
    if dtype == "bf16":
        b = x.view(np.uint32)
        lower = b & 0xFFFF
        upper = b >> 16
        up = (lower > 0x8000) | ((lower == 0x8000) & ((upper & 1) == 1))
        return ((upper + up) & 0xFFFF).astype(np.uint16)
    return x.copy()


def _normal(rng, shape, sigma=1.0, mean=0.0):
    x = rng.standard_normal(shape, dtype=np.float32)
    if sigma != 1.0:
        x *= np.float32(sigma)
    if mean != 0.0:
        x += np.float32(mean)
    return x


def zipf_ids(rng, n: int, vocab: int, s: float) -> np.ndarray:
    """Finite Zipf: rank k in [1, vocab] with p(k) proportional to k^-s; id = k - 1."""
    k = np.arange(1, vocab + 1, dtype=np.float64)
    p = k ** (-s)
    cdf = np.cumsum(p)
    cdf /= cdf[-1]
    u = rng.random(n)
    return np.minimum(np.searchsorted(cdf, u, side="right"), vocab - 1).astype(np.int32)


def positions(rng, cfg: LayerConfig) -> np.ndarray:
    if cfg.positions == "arange":
        return np.arange(cfg.T, dtype=np.int32)
    hi = int(cfg.positions.split(":")[1])
    return rng.integers(0, hi, cfg.T, dtype=np.int64).astype(np.int32)


def make_layer_inputs(cfg: LayerConfig, seed: int = 0, with_table: bool = True) -> dict[str, np.ndarray]:
    """Draw order: x, residual, w_attn, w_ffn, gate, up, q, k, positions,
    table, ids (table and ids only when with_table)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    T, H, I = cfg.T, cfg.H, cfg.I
    d = {}
    d["x"] = round_to(_normal(rng, (T, H)), cfg.dtype)
    d["residual"] = round_to(_normal(rng, (T, H), cfg.res_sigma), cfg.dtype)
    d["w_attn"] = round_to(_normal(rng, (H,), 0.02, 1.0), cfg.dtype)
    d["w_ffn"] = round_to(_normal(rng, (H,), 0.02, 1.0), cfg.dtype)
    d["gate"] = round_to(_normal(rng, (T, I), cfg.gate_sigma), cfg.dtype)
    d["up"] = round_to(_normal(rng, (T, I), cfg.gate_sigma), cfg.dtype)
    d["q"] = round_to(_normal(rng, (T, cfg.nq, cfg.D)), cfg.dtype)
    d["k"] = round_to(_normal(rng, (T, cfg.nkv, cfg.D)), cfg.dtype)
    d["pos"] = positions(rng, cfg)
    if with_table:
        d["table"] = round_to(_normal(rng, (cfg.vocab, H), 0.02), cfg.dtype)
        if cfg.ids.startswith("zipf"):
            d["ids"] = zipf_ids(rng, T, cfg.vocab, float(cfg.ids.split(":")[1]))
        else:
            d["ids"] = rng.integers(0, cfg.vocab, T, dtype=np.int64).astype(np.int32)
    return d


def make_quant_inputs(seed: int = 0, T: int = QUANT_T, H: int = QUANT_H, wn: int = QUANT_WN,
                      wk: int = QUANT_WK) -> dict[str, np.ndarray]:
    """Draw order: activations Student-t(3) [T, H], outlier channels (0.1% of H,
    scaled x20), norm weight N(1, 0.02), int8 weights U{-127..127} [wn, wk],
    per-row fp16 scales U(1e-3, 1e-2) widened exactly to fp32."""
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_t(3.0, (T, H)).astype(np.float32)
    n_out = max(1, H // 1000)
    ch = rng.choice(H, n_out, replace=False)
    x[:, ch] *= np.float32(20.0)
    d = {"x": round_to(x, "f16"), "outlier_channels": np.sort(ch).astype(np.int32)}
    d["w"] = round_to(_normal(rng, (H,), 0.02, 1.0), "f16")
    d["wq"] = rng.integers(-127, 128, (wn, wk), dtype=np.int64).astype(np.int8)
    sc16 = rng.uniform(1e-3, 1e-2, wn).astype(np.float16)
    d["wscale"] = sc16.astype(np.float32)
    return d


def layer_bytes(cfg: LayerConfig) -> dict[str, int]:
    """Algorithmic bytes per kernel for one decoder layer (and gather per forward)."""
    T, H, I, D, e = cfg.T, cfg.H, cfg.I, cfg.D, cfg.e
    return {
        "rmsnorm": 2 * T * H * e + H * e,
        "rope_q": 2 * T * cfg.nq * D * e + 4 * T,
        "rope_k": 2 * T * cfg.nkv * D * e + 4 * T,
        "add_rmsnorm": 4 * T * H * e + H * e,
        "silu_mul": 3 * T * I * e,
        "add": 3 * T * H * e,
        "gather": 2 * T * H * e + 4 * T,
    }


LAYER_KERNELS = ("rmsnorm", "rope_q", "rope_k", "add_rmsnorm", "silu_mul", "add")


def quant_bytes(T: int = QUANT_T, H: int = QUANT_H, wn: int = QUANT_WN, wk: int = QUANT_WK) -> dict[str, int]:
    return {
        "rmsnorm_quant": T * H * 2 + T * H + 4 * T + H * 2,
        "quant_per_token": T * H * 2 + T * H + 4 * T,
        "dequant": wn * wk + 4 * wn + 2 * wn * wk,
    }
