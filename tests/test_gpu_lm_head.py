"""lm_head logits and the greedy token against the oracle.

Logits: the oracle's float64 dot product rounded once; the kernel must give
the same float32 value (at most one unit in the last place apart, for the
rare sums that fall within a float64 rounding of a float32 tie; counted and
bounded).  Token: bit-exact argmax of nan_to_num with the first index on
ties, checked against the oracle applied to the kernel's own logits and, at
the gpt-oss vocabulary, to the oracle's logits.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from klcquant_amd import _native
from klcquant_amd.lm_head import LmHead
from oracle import lm_head as olm
from oracle.numerics import f32_to_bf16

pytestmark = pytest.mark.gpu


def _weights(rng, vocab, hidden, scale=0.02):
    return f32_to_bf16((rng.standard_normal((vocab, hidden)) * scale).astype(np.float32))


def _check(gpu, w_bits, x, expect_token_unique=True):
    w = torch.from_numpy(w_bits.view(np.int16)).view(torch.bfloat16).to(gpu)
    head = LmHead(w)
    got, token = head.logits_device(torch.from_numpy(x).to(gpu))
    got = got.cpu().numpy()
    want = olm.logits(w_bits, x)
    both_nan = np.isnan(got) & np.isnan(want)
    same = (got.view(np.uint32) == want.view(np.uint32)) | both_nan
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert (same | (np.isfinite(want) & (ulp <= 1))).all()
    assert (~same).sum() <= max(2, got.size // 100000)
    t = int(token.item())
    assert t == olm.greedy_token(got)
    if expect_token_unique:
        assert t == olm.greedy_token(want)
    return head, got, t


@pytest.mark.parametrize("vocab,hidden", [(1, 8), (7, 64), (1000, 520), (12345, 2880), (3001, 4096), (257, 8)])
def test_logits_and_token_match_oracle(gpu, vocab, hidden):
    rng = np.random.default_rng(vocab * 7 + hidden)
    _check(gpu, _weights(rng, vocab, hidden), rng.standard_normal(hidden).astype(np.float32))


def test_nan_inf_and_ties(gpu):
    """NaN and +-inf logits rank as nan_to_num maps them; equal maxima go to
    the first index."""
    rng = np.random.default_rng(3)
    vocab, hidden = 4099, 128
    w = _weights(rng, vocab, hidden, 0.01)
    x = rng.standard_normal(hidden).astype(np.float32)
    nan, inf = np.uint16(0x7FC0), np.uint16(0x7F80)
    w[10, 5] = nan                      # NaN logit -> -1e9
    w[11, :] = 0; w[11, 3] = inf; x[3] = abs(x[3]) + 1  # +inf logit -> 1e9: the winner
    w[12, :] = 0; w[12, 4] = inf; x[4] = -(abs(x[4]) + 1)  # -inf -> -1e9
    w[4000] = w[11]                     # a later +inf: the first one wins
    _, got, t = _check(gpu, w, x)
    assert np.isnan(got[10]) and got[11] == np.inf and got[12] == -np.inf and t == 11
    # all-equal rows: the first index
    _check(gpu, np.tile(_weights(rng, 1, hidden), (777, 1)), x)


def test_gpt_oss_vocabulary(gpu):
    """201,088 x 2880: every row against the oracle, and the token."""
    rng = np.random.default_rng(5)
    vocab, hidden = 201088, 2880
    w_bits = np.empty((vocab, hidden), dtype=np.uint16)
    for s in range(0, vocab, 16384):
        w_bits[s:s + 16384] = _weights(rng, min(16384, vocab - s), hidden)
    x = rng.standard_normal(hidden).astype(np.float32)
    head, got, t = _check(gpu, w_bits, x)
    cpu = head.logits(torch.from_numpy(x).to(gpu), chunk_rows=4096)
    assert cpu.device.type == "cpu" and cpu.dtype == torch.float32 and np.array_equal(cpu.numpy(), got)
    assert head.greedy_token(torch.from_numpy(x).to(gpu)) == t


def test_rejects_bad_arguments(gpu):
    w = torch.zeros((16, 12), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(_native.KlcError) as exc:
        LmHead(w).logits_device(torch.zeros(12, device=gpu))
    assert exc.value.status == -3  # hidden not a multiple of 8
    w = torch.zeros((16, 16), dtype=torch.bfloat16, device=gpu)
    x = torch.zeros(16, device=gpu)
    out = torch.empty(16, device=gpu)
    tok = torch.empty(1, dtype=torch.int32, device=gpu)
    ws = torch.empty(64, dtype=torch.uint8, device=gpu)
    with pytest.raises(_native.KlcError) as exc:
        _native.call("klc_lm_head_logits", ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                     ctypes.c_void_p(out.data_ptr()), 16, 16, ctypes.c_void_p(ws.data_ptr()), 8,
                     ctypes.c_void_p(tok.data_ptr()), None, None)
    assert exc.value.status == -1  # workspace too small
    with pytest.raises(ValueError):
        LmHead(w.float())
