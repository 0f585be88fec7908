"""The attention oracle pinned by closed forms and by torch's own bf16 op
semantics (the functions the reference calls), not by restating it."""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import attention as oat
from oracle.numerics import bf16_to_f32, f32_to_bf16


def test_yarn_without_scaling_is_plain_rope():
    inv = oat.yarn_inv_freq(64, 150000.0, 1.0, 4096, 32.0, 1.0)
    assert np.allclose(inv, 150000.0 ** (-np.arange(0, 64, 2) / 64), rtol=1e-15)


def test_yarn_ramp_ends():
    """Dimensions below the fast correction keep the original frequency,
    those above the slow one are divided by the factor (gpt-oss: factor 32)."""
    inv = oat.yarn_inv_freq(64, 150000.0, 32.0, 4096, 32.0, 1.0)
    plain = 150000.0 ** (-np.arange(0, 64, 2) / 64)
    low = 64 * math.log(4096 / (32 * 2 * math.pi)) / (2 * math.log(150000.0))
    high = 64 * math.log(4096 / (1 * 2 * math.pi)) / (2 * math.log(150000.0))
    i = np.arange(32)
    assert np.allclose(inv[i <= low], plain[i <= low], rtol=1e-15)
    assert np.allclose(inv[i >= high], plain[i >= high] / 32.0, rtol=1e-15)
    assert (inv[(i > low) & (i < high)] < plain[(i > low) & (i < high)]).all()
    assert math.isclose(oat.attention_scaling(32.0), 0.1 * math.log(32.0) + 1.0)


def test_rope_matches_torch_bf16_ops():
    rng = np.random.default_rng(4)
    x = f32_to_bf16(rng.standard_normal((64, 64)).astype(np.float32))
    ang = rng.uniform(0, 6.3, 32).astype(np.float32)
    c, s = f32_to_bf16(np.cos(ang)), f32_to_bf16(np.sin(ang))
    tx = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    tc = torch.from_numpy(c.view(np.int16)).view(torch.bfloat16)
    ts = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16)
    a, b = torch.chunk(tx, 2, dim=-1)
    want = torch.cat((a * tc - b * ts, b * tc + a * ts), dim=-1).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oat.rope_rotate(x, c, s), want)
    one, zero = f32_to_bf16(np.ones(32, np.float32)), f32_to_bf16(np.zeros(32, np.float32))
    assert np.array_equal(oat.rope_rotate(x, one, zero), x)


def test_single_key_with_sink_is_logistic():
    rng = np.random.default_rng(5)
    q = f32_to_bf16(rng.standard_normal((8, 64)).astype(np.float32))
    k = f32_to_bf16(rng.standard_normal((1, 2, 64)).astype(np.float32))
    v = f32_to_bf16(rng.standard_normal((1, 2, 64)).astype(np.float32))
    sinks = f32_to_bf16(rng.standard_normal(8).astype(np.float32))
    ctx, probs = oat.decode_attention(q, k, v, sinks)
    qf, kf = bf16_to_f32(q).astype(np.float64), np.repeat(bf16_to_f32(k)[0], 4, axis=0).astype(np.float64)
    s = (qf * kf).sum(1) / 8.0
    p = 1.0 / (1.0 + np.exp(bf16_to_f32(sinks) - s))
    assert np.allclose(probs[:, 0], p, rtol=2 ** -7)
    _, probs_nosink = oat.decode_attention(q, k, v, None)
    assert (probs_nosink == 1.0).all()
    _, probs16 = oat.decode_attention(q, k, v, sinks, kv="fp16")
    assert np.allclose(probs16[:, 0], p, rtol=2 ** -10)


def test_matches_torch_float32_formula():
    """torch float32 einsum/softmax (the reference's ops) within their rounding."""
    rng = np.random.default_rng(6)
    t, nh, nkv, d = 300, 64, 8, 64
    q = f32_to_bf16(rng.standard_normal((nh, d)).astype(np.float32))
    k = f32_to_bf16(rng.standard_normal((t, nkv, d)).astype(np.float32))
    v = f32_to_bf16(rng.standard_normal((t, nkv, d)).astype(np.float32))
    sinks = f32_to_bf16(rng.standard_normal(nh).astype(np.float32))
    ctx, _ = oat.decode_attention(q, k, v, sinks, window=128)
    tq = torch.from_numpy(bf16_to_f32(q))
    tk = torch.from_numpy(bf16_to_f32(k[-128:])).repeat_interleave(8, dim=1).transpose(0, 1)
    tv = torch.from_numpy(bf16_to_f32(v[-128:])).repeat_interleave(8, dim=1).transpose(0, 1)
    scores = torch.einsum("hd,htd->ht", tq, tk) / math.sqrt(d)
    comb = torch.cat([scores, torch.from_numpy(bf16_to_f32(sinks)).reshape(-1, 1)], dim=-1)
    comb = comb - comb.max(dim=-1, keepdim=True).values
    probs = torch.softmax(comb, dim=-1)[..., :-1].to(torch.bfloat16).float()
    want = torch.einsum("ht,htd->hd", probs, tv).numpy()
    got = bf16_to_f32(ctx)
    assert np.allclose(got, want, rtol=2e-2, atol=1e-2)
