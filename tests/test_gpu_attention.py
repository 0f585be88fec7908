"""Decode attention on the device KV ring against the oracle.

Cases cover the single-split path (at most 256 keys) and the split path
with its statistics and combine launches (up to 4500 keys, 18 splits).  RoPE
and the stored keys/values are bit-exact (every bfloat16 op rounded as
torch rounds it, then the cache type's rounding); the context is within a
few cache-type ulps of |ref| plus 2^-9 of the head's largest |ref| of the
oracle (probabilities rounded to the cache type can land one unit apart when
the softmax sum is taken in another order).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from klcquant_amd import _native
from klcquant_amd.attention import AttentionConfig, DeviceKVCache, StreamedAttention, rope_cos_sin
from oracle import attention as oat
from oracle.numerics import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu
P = ctypes.c_void_p
CFG = dict(hidden_size=2880, num_heads=64, num_kv_heads=8, head_dim=64, rope_theta=150000.0, rope_factor=32.0,
           rope_beta_fast=32.0, rope_beta_slow=1.0, rope_original_max_position_embeddings=4096)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def dev(b: np.ndarray, gpu) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(gpu)


def context_tolerance(ref: np.ndarray, kv: str) -> np.ndarray:
    """Per-element bound for the context [heads, head_dim]: the context is rounded twice (cache
    type, then bfloat16) and a probability rounded to the cache type may land one unit off, which
    moves the head's weighted sum by at most that unit times its largest values; so a few cache-type
    ulps of |ref| plus 2^-9 of the head's largest |ref|."""
    ulp = 2.0 ** -10 if kv == "fp16" else 2.0 ** -7
    head_max = np.abs(ref).max(axis=-1, keepdims=True)
    return 4 * ulp * np.abs(ref) + 2.0 ** -8 * np.abs(ref) + 2.0 ** -9 * head_max


@pytest.mark.parametrize("kv", ["fp16", "bf16"])
@pytest.mark.parametrize("steps,cap,window,sinks", [(1, 64, None, True), (300, 512, None, True), (300, 512, 128, False),
                                                    (700, 512, None, True), (700, 1024, None, False),
                                                    (1000, 1024, 128, True), (4500, 8192, None, True),
                                                    (4500, 8192, None, False)])
def test_rope_append_and_decode_match_oracle(gpu, kv, steps, cap, window, sinks):
    cfg = AttentionConfig(**CFG)
    nh, nkv, d = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    rng = np.random.default_rng(steps * 3 + cap + (window or 0) + len(kv))
    code = 1 if kv == "fp16" else 0
    kdt = torch.float16 if kv == "fp16" else torch.bfloat16
    kc = torch.empty((cap, nkv, d), dtype=kdt, device=gpu)
    vc = torch.empty((cap, nkv, d), dtype=kdt, device=gpu)
    keys_rot, vals = [], []
    stream = P(torch.cuda.current_stream(gpu).cuda_stream)
    for pos in range(steps):
        q = f32_to_bf16(rng.standard_normal((nh, d)).astype(np.float32))
        k = f32_to_bf16(rng.standard_normal((nkv, d)).astype(np.float32))
        v = f32_to_bf16(rng.standard_normal((nkv, d)).astype(np.float32))
        cos, sin = rope_cos_sin(cfg, pos, gpu, torch.bfloat16)
        qd, kd, vd = dev(q, gpu), dev(k, gpu), dev(v, gpu)
        q_out, k_out = torch.empty_like(qd), torch.empty_like(kd)
        _native.call("klc_rope_append", P(qd.data_ptr()), P(kd.data_ptr()), P(vd.data_ptr()), P(cos.data_ptr()),
                     P(sin.data_ptr()), P(q_out.data_ptr()), P(k_out.data_ptr()), P(kc.data_ptr()), P(vc.data_ptr()),
                     pos % cap, cap, nh, nkv, d, code, stream)
        cb, sb = bits(cos), bits(sin)
        k_rot = oat.rope_rotate(k, cb, sb)
        keys_rot.append(k_rot)
        vals.append(v)
    q_rot = oat.rope_rotate(q, cb, sb)
    assert np.array_equal(bits(q_out), q_rot) and np.array_equal(bits(k_out), k_rot)
    slot = (steps - 1) % cap
    assert np.array_equal(kc[slot].float().cpu().numpy(), oat.to_kv(bf16_to_f32(k_rot), kv))
    assert np.array_equal(vc[slot].float().cpu().numpy(), oat.to_kv(bf16_to_f32(v), kv))
    held = min(steps, cap)
    count = min(held, window) if window else held
    first = (steps - count) % cap
    sk = f32_to_bf16(rng.standard_normal(nh).astype(np.float32)) if sinks else None
    skd = dev(sk, gpu) if sinks else None
    ws = torch.empty(_native.call("klc_attn_workspace_bytes", nh, d, count), dtype=torch.uint8, device=gpu)
    ctx = torch.empty((nh, d), dtype=torch.bfloat16, device=gpu)
    _native.call("klc_attn_decode", P(q_out.data_ptr()), P(kc.data_ptr()), P(vc.data_ptr()),
                 P(0 if skd is None else skd.data_ptr()), cap, first, count, nh, nkv, d, code, P(ws.data_ptr()),
                 ws.numel(), P(ctx.data_ptr()), stream)
    want, _ = oat.decode_attention(q_rot, np.stack(keys_rot[-count:]), np.stack(vals[-count:]), sk, kv=kv)
    got, ref = bf16_to_f32(bits(ctx)), bf16_to_f32(want)
    assert np.all(np.abs(got - ref) <= context_tolerance(ref, kv)), np.abs(got - ref).max()


@pytest.mark.parametrize("kv", ["fp16", "bf16"])
def test_streamed_attention_forward_matches_oracle(gpu, kv):
    """Eight decode steps through StreamedAttention.forward (sliding window 4):
    torch's projections, then the oracle's RoPE and attention."""
    cfg = AttentionConfig(**CFG, sliding_window=4)
    nh, nkv, d, h = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.hidden_size
    g = torch.Generator(device=gpu).manual_seed(11)
    pre = "model.layers.0.self_attn"

    def w(*s, scale=0.02):
        return (torch.randn(s, generator=g, device=gpu) * scale).to(torch.bfloat16)

    tensors = {f"{pre}.q_proj.weight": w(nh * d, h), f"{pre}.q_proj.bias": w(nh * d),
               f"{pre}.k_proj.weight": w(nkv * d, h), f"{pre}.k_proj.bias": w(nkv * d),
               f"{pre}.v_proj.weight": w(nkv * d, h), f"{pre}.v_proj.bias": w(nkv * d),
               f"{pre}.o_proj.weight": w(h, nh * d), f"{pre}.o_proj.bias": w(h), f"{pre}.sinks": w(nh, scale=1.0)}
    attn, cache = StreamedAttention(cfg), DeviceKVCache(gpu, precision=kv, capacity=4)
    keys, vals = [], []
    lin = torch.nn.functional.linear
    for pos in range(8):
        x = w(h, scale=1.0)
        out, diag = attn.forward(0, x, tensors, pos, cache)
        q = bits(lin(x, tensors[f"{pre}.q_proj.weight"], tensors[f"{pre}.q_proj.bias"]).view(nh, d))
        k = bits(lin(x, tensors[f"{pre}.k_proj.weight"], tensors[f"{pre}.k_proj.bias"]).view(nkv, d))
        v = bits(lin(x, tensors[f"{pre}.v_proj.weight"], tensors[f"{pre}.v_proj.bias"]).view(nkv, d))
        cos, sin = rope_cos_sin(cfg, pos, gpu, torch.bfloat16)
        q_rot, k_rot = oat.rope_rotate(q, bits(cos), bits(sin)), oat.rope_rotate(k, bits(cos), bits(sin))
        keys.append(k_rot)
        vals.append(v)
        ctx, _ = oat.decode_attention(q_rot, np.stack(keys[-4:]), np.stack(vals[-4:]), bits(tensors[f"{pre}.sinks"]), kv=kv)
        want = lin(dev(ctx, gpu).reshape(-1), tensors[f"{pre}.o_proj.weight"], tensors[f"{pre}.o_proj.bias"]).float()
        assert torch.allclose(out.float(), want, rtol=2e-2, atol=1e-2)
        assert diag["rope_position"] == pos and diag["q_post_rope_nonfinite_count"] == 0
        assert np.isclose(diag["k_post_rope_norm"], np.linalg.norm(bf16_to_f32(k_rot)), rtol=1e-5)
    assert cache.stats().tokens == 8 and cache.get(0, 4)[0].shape == (4, nkv, d)


def test_device_kv_cache_api(gpu):
    """append/get/max_tokens/snapshot/restore as kv_cache_manager.py:39-97 keep them."""
    c = DeviceKVCache(gpu, max_tokens=3, precision="bf16")
    ks = [torch.full((2, 8), float(i), dtype=torch.bfloat16, device=gpu) for i in range(5)]
    for i, k in enumerate(ks):
        c.append(1, k, -k)
    keys, values = c.get(1)
    assert keys[:, 0, 0].tolist() == [2.0, 3.0, 4.0] and values[:, 0, 0].tolist() == [-2.0, -3.0, -4.0]
    assert c.get(1, window=2)[0][:, 0, 0].tolist() == [3.0, 4.0] and c.get(7) == (None, None)
    assert c.stats().tokens == 3 and c.stats().resident_bytes == 2 * 3 * 16 * 2
    snap = c.snapshot()
    c.clear()
    assert c.get(1) == (None, None)
    c.restore(snap)
    assert c.get(1)[0][:, 0, 0].tolist() == [2.0, 3.0, 4.0]
    g = DeviceKVCache(gpu, precision="fp16", capacity=2)  # unbounded: grows past its capacity
    for i, k in enumerate(ks):
        g.append(0, k, k)
    assert g.get(0)[0].dtype == torch.float16 and g.get(0)[0][:, 0, 0].tolist() == [0.0, 1.0, 2.0, 3.0, 4.0]
    with pytest.raises(ValueError):
        DeviceKVCache(gpu, precision="q8")


@pytest.mark.parametrize("nh,nkv,d", [(32, 2, 128), (8, 8, 8), (12, 4, 24)])
@pytest.mark.parametrize("window", [None, 100])
def test_other_head_shapes(gpu, nh, nkv, d, window):
    """Group sizes 16, 1 and 3 and head dims 128, 8 and 24 (a value-slice
    count that does not divide the workgroup), bf16 cache, 300 steps."""
    cfg = AttentionConfig(hidden_size=nh * d, num_heads=nh, num_kv_heads=nkv, head_dim=d, rope_factor=8.0)
    rng = np.random.default_rng(nh * 1000 + d + (window or 0))
    cap, steps = 512, 300
    kc = torch.empty((cap, nkv, d), dtype=torch.bfloat16, device=gpu)
    vc = torch.empty((cap, nkv, d), dtype=torch.bfloat16, device=gpu)
    stream = P(torch.cuda.current_stream(gpu).cuda_stream)
    keys, vals = [], []
    for pos in range(steps):
        q = f32_to_bf16(rng.standard_normal((nh, d)).astype(np.float32))
        k = f32_to_bf16(rng.standard_normal((nkv, d)).astype(np.float32))
        v = f32_to_bf16(rng.standard_normal((nkv, d)).astype(np.float32))
        cos, sin = rope_cos_sin(cfg, pos, gpu, torch.bfloat16)
        qd, kd, vd = dev(q, gpu), dev(k, gpu), dev(v, gpu)
        q_out = torch.empty_like(qd)
        _native.call("klc_rope_append", P(qd.data_ptr()), P(kd.data_ptr()), P(vd.data_ptr()), P(cos.data_ptr()),
                     P(sin.data_ptr()), P(q_out.data_ptr()), None, P(kc.data_ptr()), P(vc.data_ptr()), pos % cap,
                     cap, nh, nkv, d, 0, stream)
        keys.append(oat.rope_rotate(k, bits(cos), bits(sin)))
        vals.append(v)
    q_rot = oat.rope_rotate(q, bits(cos), bits(sin))
    assert np.array_equal(bits(q_out), q_rot)
    count = min(steps, window) if window else steps
    sk = f32_to_bf16(rng.standard_normal(nh).astype(np.float32))
    skd = dev(sk, gpu)
    ws = torch.empty(_native.call("klc_attn_workspace_bytes", nh, d, count), dtype=torch.uint8, device=gpu)
    ctx = torch.empty((nh, d), dtype=torch.bfloat16, device=gpu)
    _native.call("klc_attn_decode", P(q_out.data_ptr()), P(kc.data_ptr()), P(vc.data_ptr()), P(skd.data_ptr()), cap,
                 steps - count, count, nh, nkv, d, 0, P(ws.data_ptr()), ws.numel(), P(ctx.data_ptr()), stream)
    want, _ = oat.decode_attention(q_rot, np.stack(keys[-count:]), np.stack(vals[-count:]), sk, kv="bf16")
    got, ref = bf16_to_f32(bits(ctx)), bf16_to_f32(want)
    assert np.all(np.abs(got - ref) <= context_tolerance(ref, "bf16")), np.abs(got - ref).max()


def test_attention_rejects_bad_shapes(gpu):
    x = torch.zeros(4096, dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(1 << 16, dtype=torch.uint8, device=gpu)
    stream = P(torch.cuda.current_stream(gpu).cuda_stream)

    def decode(nh, nkv, d, count=4, cap=8, first=0):
        with pytest.raises(_native.KlcError) as exc:
            _native.call("klc_attn_decode", P(x.data_ptr()), P(x.data_ptr()), P(x.data_ptr()), None, cap, first,
                         count, nh, nkv, d, 0, P(ws.data_ptr()), ws.numel(), P(x.data_ptr()), stream)
        return exc.value.status

    assert decode(34, 2, 64) == -2      # group of 17 > 16
    assert decode(8, 8, 136) == -2      # head_dim above 128
    assert decode(8, 8, 12) == -2       # head_dim not a multiple of 8
    assert decode(8, 3, 64) == -2       # heads not a multiple of KV heads
    assert decode(8, 8, 64, count=9) == -1   # more keys than the ring holds
    assert decode(8, 8, 64, first=8) == -1   # first slot outside the ring
    with pytest.raises(_native.KlcError) as exc:
        _native.call("klc_rope_append", P(x.data_ptr()), P(x.data_ptr()), P(x.data_ptr()), P(x.data_ptr()),
                     P(x.data_ptr()), P(x.data_ptr()), None, P(x.data_ptr()), P(x.data_ptr()), 8, 8, 8, 8, 64, 0,
                     stream)
    assert exc.value.status == -1       # slot == cap
