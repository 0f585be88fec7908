"""Measurement: the scaled FP4 MFMA (v_mfma_scale_f32_16x16x128_f8f6f4) against exact sums.

The grouped expert GEMMs decode E2M1 codes in registers into bf16 MFMA
operands, which keeps every product exact and the sums in float32.  The
scaled FP4 MFMA would take the checkpoint's codes and scales as they are, with
the activations as FP8 E4M3 planes.  These tests run that instruction
(tests/native/libfp4_mfma_probe.so) and report

* per 128-term block: |error| / sum |terms| against the exact sum, with unit
  and with mixed E8M0 scales, every input exactly representable;
* one 120B-shaped expert (2880 -> 5760 -> SwiGLU -> 2880) over 256 tokens of
  bf16 activations split into 1, 2 or 3 FP8 planes: the elements that fail
  the expert-output tolerance (1e-2 + 2e-2 |ref|) against the oracle.

They assert only what makes the figures trustworthy (the operand layout is
right: a wrong lane, nibble or scale mapping gives errors of order 1) and
print the measurements (run with ``-s``).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

import mx_operands as mx
from klcquant_amd import synth
from oracle import experts as oex
from oracle import mxfp4 as omx
from oracle.numerics import bf16_to_f32

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "native" / "libfp4_mfma_probe.so"
HIDDEN, INTER, TOKENS = 2880, 2880, 256
RTOL, ATOL = 2e-2, 1e-2


@pytest.fixture(scope="module")
def probe(gpu):
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (build() compiles tests/native/*.hip)")
    so = ctypes.CDLL(str(LIB))
    so.fp4_fp8_gemm.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 4 + [ctypes.c_void_p] * 2
    so.fp4_fp8_gemm.restype = ctypes.c_int
    return so


def run_gemm(so, dev, blocks, a_scales, codes, b_scales) -> np.ndarray:
    """``[n, rows]`` float32: rows of MXFP4 ``blocks/a_scales`` times the FP8 planes ``codes/b_scales``."""
    ac, asc, steps = mx.pack_a(blocks, a_scales)
    bc, bsc = mx.pack_b(codes, b_scales, steps)
    rows, n, planes = blocks.shape[0], codes.shape[1], codes.shape[0]
    t = [torch.from_numpy(v).to(dev) for v in (ac, asc, bc, bsc)]
    out = torch.empty((n, rows), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = so.fp4_fp8_gemm(*(v.data_ptr() for v in t), rows // 16, n // 16, steps, planes, out.data_ptr(), stream)
    assert rc == 0
    torch.cuda.synchronize(dev)
    return out.cpu().numpy()


@pytest.mark.parametrize("scale_lo,scale_hi", [(127, 127), (120, 134)])
def test_block_error_against_exact_sums(probe, gpu, scale_lo, scale_hi):
    """65536 sums of 128 exactly representable products, one MFMA each."""
    rng = np.random.default_rng(1000 + scale_lo)
    rows, n = 256, 256
    blocks = rng.integers(0, 256, (rows, 4, 16), dtype=np.uint8)
    a_sc = rng.integers(scale_lo, scale_hi + 1, (rows, 4)).astype(np.uint8)
    codes = rng.integers(0, 256, (1, n, 128), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x7E  # no NaN codes
    b_sc = rng.integers(scale_lo, scale_hi + 1, (1, n, 4)).astype(np.uint8)
    got = run_gemm(probe, gpu, blocks, a_sc, codes, b_sc).astype(np.float64)
    exact, mag = mx.exact_block_sums(blocks, a_sc, codes[0], b_sc[0], min(scale_lo, 120))
    rel = np.abs(got - exact) / np.where(mag > 0, mag, 1.0)
    # what a float32 sum of the same terms in k order loses, for comparison
    a_val = omx.dequant_values_f32(blocks, a_sc).astype(np.float32)
    b_val = (mx.e4m3_values()[codes[0]].reshape(n, 4, 32) * np.ldexp(1.0, b_sc[0].astype(int) - 127)[..., None])
    b_val = b_val.reshape(n, 128).astype(np.float32)
    seq = np.zeros((n, rows), np.float32)
    for k in range(128):
        seq = seq + b_val[:, k:k + 1] * a_val[None, :, k]
    rel32 = np.abs(seq.astype(np.float64) - exact) / np.where(mag > 0, mag, 1.0)
    worst = np.unravel_index(np.argmax(rel), rel.shape)
    print(f"\nscaled FP4 MFMA, one 128-term block, E8M0 scales {scale_lo}..{scale_hi}: |err|/sum|terms| "
          f"max {rel.max():.3e} (2^{np.log2(max(rel.max(), 1e-300)):.1f}), p99.9 {np.quantile(rel, 0.999):.3e}, "
          f"median {np.median(rel):.3e}, exact {np.mean(rel == 0):.1%}; float32 sequential sum: max "
          f"{rel32.max():.3e}, median {np.median(rel32):.3e}; worst block token {worst[0]} row {worst[1]}: "
          f"exact {exact[worst]:.9g} got {got[worst]:.9g} sum|terms| {mag[worst]:.6g}")
    assert rel.max() < 1e-3, "operand layout or scale mapping is wrong"


def exact_gemm(blocks, a_scales, codes, b_scales) -> np.ndarray:
    """The same product with exact float64 sums, rounded once to float32: what the planes alone cost."""
    a = omx.dequant_values_f32(blocks, a_scales).astype(np.float64)
    return (mx.plane_values(codes, b_scales) @ a.T).astype(np.float32)


def expert_chain(gemm, x_bits, gub, gus, gu_bias, db, ds, d_bias, planes):
    x = bf16_to_f32(x_bits).astype(np.float64)
    c, s, _ = mx.fp8_planes(x, planes)
    gu = gemm(gub, gus, c, s) + bf16_to_f32(gu_bias)[None, :]
    gated = oex.swiglu(gu)
    c, s, _ = mx.fp8_planes(gated.astype(np.float64), planes)
    return gemm(db, ds, c, s) + bf16_to_f32(d_bias)[None, :]


def test_expert_outputs_with_fp8_planes(probe, gpu):
    """One expert of the 120B shape, synthetic weights (expert 0 of the seeded 120B layer), 256 tokens.
    Each plane count runs twice: through the MFMA, and with exact sums of the same planes."""
    wl = 2
    gub, gus = synth.mxfp4_expert_slice(synth.tensor_seed(wl, "gate_up_blocks"), synth.tensor_seed(wl, "gate_up_scales"),
                                        0, 2 * INTER, HIDDEN)
    db, ds = synth.mxfp4_expert_slice(synth.tensor_seed(wl, "down_blocks"), synth.tensor_seed(wl, "down_scales"), 0,
                                      HIDDEN, INTER)
    gu_bias = synth.random_normal_bf16(synth.tensor_seed(wl, "gate_up_bias"), 2 * INTER, 0.0, 0.01)
    d_bias = synth.random_normal_bf16(synth.tensor_seed(wl, "down_bias"), HIDDEN, 0.0, 0.01)
    x_bits = synth.random_normal_bf16(synth.tensor_seed(wl, "hidden"), TOKENS * HIDDEN).reshape(TOKENS, HIDDEN)
    gu_w = omx.dequantize(gub, gus, "f32")
    d_w = omx.dequantize(db, ds, "f32")
    gated_ref, ref = oex.expert_ffn(bf16_to_f32(x_bits), gu_w, gu_bias, d_w, d_bias)
    ref = ref.astype(np.float64)
    mag = np.abs(gated_ref.astype(np.float64)) @ np.abs(d_w.astype(np.float64))
    mfma = lambda b, sc, c, cs: run_gemm(probe, gpu, b, sc, c, cs)  # noqa: E731
    lines = []
    for planes in (1, 2, 3):
        for name, gemm in (("scaled MFMA", mfma), ("exact sums ", exact_gemm)):
            got = expert_chain(gemm, x_bits, gub, gus, gu_bias, db, ds, d_bias, planes).astype(np.float64)
            err = np.abs(got - ref)
            over = err - (ATOL + RTOL * np.abs(ref))
            bad = np.argwhere(over > 0)
            rel = err / np.maximum(mag, 1e-30)
            lines.append(f"{planes} FP8 plane(s), {name}: {bad.shape[0]} of {ref.size} outputs fail "
                         f"1e-2 + 2e-2|ref|, max |err| {err.max():.3e}, max |err|/sum|terms| {rel.max():.3e}")
            for i in np.argsort(-over[tuple(bad.T)])[:4] if bad.size else []:
                t, j = bad[i]
                lines.append(f"    token {t} out {j}: ref {ref[t, j]:.6g} got {got[t, j]:.6g} "
                             f"|err| {err[t, j]:.3e} sum|terms| {mag[t, j]:.4g}")
            if planes == 3 and gemm is mfma:
                assert rel.max() < 1e-2, "three planes should follow the exact result closely"
    print("\nscaled FP4 MFMA expert chain (2880 -> 5760 -> SwiGLU -> 2880, 256 tokens):\n" + "\n".join(lines))
