"""Deterministic synthetic inputs for the MoE expert path.

The reference ships no data and no checkpoints, so every test and benchmark
builds its inputs from seeds.  The generator is counter based so that any
element can be produced independently, on the host (numpy, this module) or on
the GPU (``klc_synth_fill`` in the HIP library), with identical results:

* ``draw(seed, i)`` is the i-th output of SplitMix64 started from
  ``state = mix64(seed)``: ``mix64(state + (i + 1) * GAMMA)`` (mod 2**64).
* raw bytes: byte ``j`` of the little-endian word ``draw(seed, j // 8)``.
* integers in ``[lo, hi]``: ``lo + ((draw(seed, i) >> 32) * (hi - lo + 1)) >> 32``.
* normals: Box-Muller in float64 over ``u1 = ((d0 >> 11) + 1) * 2**-53`` and
  ``u2 = (d1 >> 11) * 2**-53`` with ``d0 = draw(seed, 2i)``,
  ``d1 = draw(seed, 2i + 1)``; rounded to float32, then to bfloat16
  (round to nearest even).

Weight distributions follow the gpt-oss-style MXFP4 synthetic workload:
E2M1 codes uniform over all 16 values (uniform bytes), E8M0 scale bytes
uniform over 118..124, activations N(0, 1), router weight N(0, 0.02), router
bias N(0, 0.01), expert biases N(0, 0.01).
"""

from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_MASK64 = (1 << 64) - 1

# Seed layout: seed = 1000 * workload + 100 * layer + tensor id.
TENSOR_IDS = {
    "hidden": 1,
    "router_weight": 2,
    "router_bias": 3,
    "gate_up_blocks": 4,
    "gate_up_scales": 5,
    "gate_up_bias": 6,
    "down_blocks": 7,
    "down_scales": 8,
    "down_bias": 9,
    "norm_weight": 10,
}


def tensor_seed(workload: int, name: str, layer: int = 0) -> int:
    return 1000 * int(workload) + 100 * int(layer) + TENSOR_IDS[name]


def mix64_int(z: int) -> int:
    """SplitMix64 finaliser on a Python int (mod 2**64)."""
    z &= _MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK64
    return z ^ (z >> 31)


def _mix64(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def draws_from_state(state: int, start: int, count: int) -> np.ndarray:
    """Outputs ``start .. start + count - 1`` of SplitMix64 begun at ``state``."""
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = np.uint64(state & _MASK64) + idx * GAMMA
    return _mix64(x)


def draws(seed: int, start: int, count: int) -> np.ndarray:
    """``draw(seed, i)`` for ``i`` in ``[start, start + count)`` as uint64."""
    return draws_from_state(mix64_int(seed), start, count)


def random_bytes(seed: int, n: int) -> np.ndarray:
    words = draws(seed, 0, (n + 7) // 8)
    return words.view(np.uint8)[:n].copy()


def random_ints(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """Integers in ``[lo, hi]`` (inclusive), one draw each, as int64."""
    span = np.uint64(hi - lo + 1)
    d = draws(seed, 0, n) >> np.uint64(32)
    with np.errstate(over="ignore"):
        v = (d * span) >> np.uint64(32)
    return v.astype(np.int64) + lo


def random_normal_f32(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    d = draws(seed, 0, 2 * n)
    d0 = d[0::2] >> np.uint64(11)
    d1 = d[1::2] >> np.uint64(11)
    u1 = (d0.astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = d1.astype(np.float64) * 2.0 ** -53
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + std * z).astype(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (nearest even); returns uint16 bit patterns.

    NaN inputs map to the canonical quiet NaN 0x7FC0 (with sign kept).
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    with np.errstate(over="ignore"):
        r = (u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)
    r = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x0040), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def random_normal_bf16(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Normals rounded to bfloat16; uint16 bit patterns."""
    return f32_to_bf16_bits(random_normal_f32(seed, n, mean, std))


def mxfp4_expert_tensors(seed_blocks: int, seed_scales: int, n_mat: int, out_dim: int, in_dim: int,
                         scale_lo: int = 118, scale_hi: int = 124) -> tuple[np.ndarray, np.ndarray]:
    """Checkpoint-layout MXFP4 tensors ``blocks[n, out, in/32, 16]`` and ``scales[n, out, in/32]``."""
    if in_dim % 32:
        raise ValueError("in_dim must be a multiple of 32")
    groups = in_dim // 32
    blocks = random_bytes(seed_blocks, n_mat * out_dim * groups * 16).reshape(n_mat, out_dim, groups, 16)
    scales = random_ints(seed_scales, n_mat * out_dim * groups, scale_lo, scale_hi).astype(np.uint8)
    return blocks, scales.reshape(n_mat, out_dim, groups)


def mxfp4_expert_slice(seed_blocks: int, seed_scales: int, expert: int, out_dim: int, in_dim: int,
                       scale_lo: int = 118, scale_hi: int = 124) -> tuple[np.ndarray, np.ndarray]:
    """Expert ``expert`` of :func:`mxfp4_expert_tensors` (``[out, in/32, 16]``, ``[out, in/32]``),
    generated alone: the counter-based stream starts at the expert's first element."""
    if in_dim % 32:
        raise ValueError("in_dim must be a multiple of 32")
    groups = in_dim // 32
    per = out_dim * groups
    words = draws(seed_blocks, expert * per * 2, per * 2)  # 16 bytes = 2 draws per (row, group)
    blocks = words.view(np.uint8).reshape(out_dim, groups, 16).copy()
    span = np.uint64(scale_hi - scale_lo + 1)
    d = draws(seed_scales, expert * per, per) >> np.uint64(32)
    with np.errstate(over="ignore"):
        scales = ((d * span) >> np.uint64(32)).astype(np.int64) + scale_lo
    return blocks, scales.astype(np.uint8).reshape(out_dim, groups)


def zipf_router_bias(x_bits: np.ndarray, w_bits: np.ndarray, k: int, s: float, seed: int) -> tuple[np.ndarray, float]:
    """bf16 router bias making expert popularity ~ Zipf(s) over a seeded permutation of the experts.

    Target pair counts are ``n_pairs * r^-s / H(E, s)`` for expert rank ``r``;
    the bias is fitted on the host (float32 logits of the actual inputs
    ``x [T, H]`` and router weight ``w [E, H]``, bf16 patterns) by 300
    multiplicative steps on ``log(count / target)``, keeping the best fit in
    L1.  Returns ``(bias bits [E], the target share of the hottest expert)``.
    """
    n_exp = w_bits.shape[0]
    perm = np.argsort(random_ints(seed, n_exp, 0, 1 << 30), kind="stable")
    rank = np.empty(n_exp, dtype=np.int64)
    rank[perm] = np.arange(1, n_exp + 1)
    p = rank.astype(np.float64) ** -s
    p /= p.sum()
    logits = bf16_bits_to_f32(x_bits) @ bf16_bits_to_f32(w_bits).T
    target = p * logits.shape[0] * k

    def counts_for(b_bits):
        top = np.argpartition(-(logits + bf16_bits_to_f32(b_bits)), k - 1, axis=1)[:, :k]
        return np.bincount(top.ravel(), minlength=n_exp)

    b = (-s * np.log(rank)).astype(np.float64)
    best, best_err = None, None
    for _ in range(300):
        bits = f32_to_bf16_bits(b.astype(np.float32))
        c = counts_for(bits)
        err = float(np.abs(c - target).sum())
        if best_err is None or err < best_err:
            best, best_err = bits, err
        b += 0.25 * (np.log(target + 0.5) - np.log(c + 0.5))
    return best, float(p.max())

