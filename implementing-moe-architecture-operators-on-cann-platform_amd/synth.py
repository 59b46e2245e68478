"""Synthetic inputs for the MoE layer: a numpy mirror of moe_synth_normal_f16 (include/moe_synth.h).

Element i of stream `stream_id` under `seed` is a pure function of (seed, stream_id, i):
    key = mix64(seed * 0x9E3779B97F4A7C15 + stream_id * 0xD1B54A32D192ED03 + 0x632BE59BD9B4E019)
    z   = mix64(key + (i + 1) * 0x9E3779B97F4A7C15)                 (mod 2^64)
    u1  = ((z >> 32) + 0.5) * 2^-32,  u2 = ((z & 0xFFFFFFFF) + 0.5) * 2^-32
    n   = sqrt(-2 ln u1) * cos(2 pi u2)                              (binary64 Box-Muller)
    out = fp16(n * sigma_i), one round-to-nearest-even from binary64
so any slice can be produced independently, on the host here or on the GPU by the library kernel.

Distributions of the BASELINE configs: x ~ N(0, 1); w_gate, W_gate, W_up ~ N(0, 1/H); W_down ~ N(0, 1/I);
for the DeepSeek-shaped config, w_gate column e is scaled by (e + 1)^-1.1 renormalised to mean 1 (Zipf).
The reference draws all of them from N(0, 1/H) with std::mt19937 (tests/moe_cpu_sim.cpp:161-167,617-625).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_MASK64 = (1 << 64) - 1

STREAM_X = 1
STREAM_W_GATE = 2
STREAM_EXPERT_WEIGHTS = 3


def _mix64_int(z: int) -> int:
    z &= _MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK64
    return z ^ (z >> 31)


def stream_key(seed: int, stream_id: int) -> int:
    return _mix64_int(seed * 0x9E3779B97F4A7C15 + stream_id * 0xD1B54A32D192ED03 + 0x632BE59BD9B4E019)


def _mix64(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def normal_f64(seed: int, stream_id: int, start: int, count: int) -> np.ndarray:
    """Unscaled binary64 normals for elements [start, start + count) of one stream."""
    key = np.uint64(stream_key(seed, stream_id))
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + 1 + count, dtype=np.uint64)
        z = _mix64(key + idx * _GOLDEN)
    u1 = ((z >> np.uint64(32)).astype(np.float64) + 0.5) * 2.0**-32
    u2 = ((z & np.uint64(0xFFFFFFFF)).astype(np.float64) + 0.5) * 2.0**-32
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)


def normal_f16(seed: int, stream_id: int, n: int, sigma_a: float, sigma_b: float | None = None,
               period: int | None = None, split: int | None = None, chunk: int = 1 << 24) -> np.ndarray:
    """fp16 samples with sigma_i = sigma_a if (i % period) < split else sigma_b (defaults: all sigma_a)."""
    out = np.empty(n, dtype=np.float16)
    for s in range(0, n, chunk):
        c = min(chunk, n - s)
        v = normal_f64(seed, stream_id, s, c)
        if period is None or sigma_b is None:
            v = v * sigma_a
        else:
            pos = np.arange(s, s + c, dtype=np.int64) % period
            v = v * np.where(pos < split, sigma_a, sigma_b)
        out[s:s + c] = v.astype(np.float16)
    return out


def zipf_column_scale(num_experts: int, s: float = 1.1) -> np.ndarray:
    """(e + 1)^-s renormalised to mean 1."""
    z = np.array([(e + 1) ** -s for e in range(num_experts)], dtype=np.float64)
    return z / z.mean()


@dataclass(frozen=True)
class MoeConfig:
    T: int
    H: int
    E: int
    K: int
    I: int
    zipf: bool = False
    name: str = ""

    @property
    def slots(self) -> int:
        return self.T * self.K


# [0] small plumbing, [1] decode target, [2] prefill, [3] Mixtral, [4] DeepSeek.
CONFIGS = {
    "small": MoeConfig(8, 64, 4, 2, 256, name="small"),
    "decode": MoeConfig(128, 2048, 16, 2, 8192, name="decode"),
    "prefill": MoeConfig(8192, 2048, 16, 2, 8192, name="prefill"),
    "mixtral": MoeConfig(4096, 4096, 8, 2, 14336, name="mixtral"),
    "deepseek": MoeConfig(16384, 2048, 64, 6, 1408, zipf=True, name="deepseek"),
}


def gen_x(cfg: MoeConfig, seed: int) -> np.ndarray:
    return normal_f16(seed, STREAM_X, cfg.T * cfg.H, 1.0).reshape(cfg.T, cfg.H)


def gen_w_gate(cfg: MoeConfig, seed: int) -> np.ndarray:
    sigma = 1.0 / math.sqrt(cfg.H)
    if not cfg.zipf:
        return normal_f16(seed, STREAM_W_GATE, cfg.H * cfg.E, sigma).reshape(cfg.H, cfg.E)
    v = normal_f64(seed, STREAM_W_GATE, 0, cfg.H * cfg.E).reshape(cfg.H, cfg.E)
    return ((v * sigma) * zipf_column_scale(cfg.E)[None, :]).astype(np.float16)


def expert_weight_sigmas(cfg: MoeConfig) -> tuple[float, float, int, int]:
    """(sigma_gate_up, sigma_down, period, split) for the flat expert_weights[E, 3I, H] tensor."""
    return 1.0 / math.sqrt(cfg.H), 1.0 / math.sqrt(cfg.I), 3 * cfg.I * cfg.H, 2 * cfg.I * cfg.H


def gen_expert_weights(cfg: MoeConfig, seed: int) -> np.ndarray:
    sa, sb, period, split = expert_weight_sigmas(cfg)
    n = cfg.E * 3 * cfg.I * cfg.H
    return normal_f16(seed, STREAM_EXPERT_WEIGHTS, n, sa, sb, period, split).reshape(cfg.E, 3 * cfg.I, cfg.H)


def gen_inputs(cfg: MoeConfig, seed: int):
    """(x [T,H], w_gate [H,E], expert_weights [E,3I,H]) as fp16 numpy arrays."""
    return gen_x(cfg, seed), gen_w_gate(cfg, seed), gen_expert_weights(cfg, seed)
