"""lm_head logits and the greedy next token on the GPU.

``LmHead`` holds the resident lm_head weight (the executor's
``lm_head_cache``, streamed_transformer_executor.py:435-455) and offers the
executor's ``logits(hidden, chunk_rows)`` (streamed_transformer_executor.py:177-209)
with the same result: float32 ``[vocab]`` on the host.  Underneath, one
klc_lm_head_logits call streams the whole weight once (no per-chunk host
copy) and also picks the greedy token of the callers
(generation_runtime.py:118-122, inference_server.py:383-386:
``argmax(nan_to_num(logits, nan=-1e9, posinf=1e9, neginf=-1e9))``), so a
decode loop can read one int instead of the whole vector.

Numerics: each logit is the correctly rounded float32 dot product (float64
accumulation of exact products); the reference's float32 matmul lies within
its own summation error of it.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native


class LmHead:
    def __init__(self, weight: torch.Tensor) -> None:
        if not isinstance(weight, torch.Tensor) or weight.device.type != "cuda":
            raise ValueError("LmHead keeps the lm_head weight in GPU memory; pass a CUDA tensor")
        if weight.dim() != 2 or weight.dtype != torch.bfloat16:
            raise ValueError(f"lm_head weight must be bfloat16 [vocab, hidden], got {weight.dtype} {tuple(weight.shape)}")
        self.weight = weight.contiguous()
        self.vocab, self.hidden = int(weight.shape[0]), int(weight.shape[1])
        self.device = weight.device
        nbytes = _native.call("klc_lm_head_workspace_bytes", self.vocab)
        self._workspace = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        self._token = torch.empty(1, dtype=torch.int32, device=self.device)
        self._token_logit = torch.empty(1, dtype=torch.float32, device=self.device)

    def logits_device(self, hidden: torch.Tensor, out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """``(logits float32 [vocab], token int32 [1])`` on the device, on the
        current stream; token = argmax(nan_to_num(logits)), first index."""
        if hidden.device != self.device or hidden.numel() != self.hidden:
            raise ValueError(f"hidden must be [{self.hidden}] on {self.device}, got {tuple(hidden.shape)} on {hidden.device}")
        x = hidden.reshape(-1).float().contiguous()
        if out is None:
            out = torch.empty(self.vocab, dtype=torch.float32, device=self.device)
        elif out.dtype != torch.float32 or out.numel() != self.vocab or out.device != self.device:
            raise ValueError(f"out must be float32 [{self.vocab}] on {self.device}")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        _native.call("klc_lm_head_logits", ctypes.c_void_p(self.weight.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                     ctypes.c_void_p(out.data_ptr()), self.vocab, self.hidden,
                     ctypes.c_void_p(self._workspace.data_ptr()), self._workspace.numel(),
                     ctypes.c_void_p(self._token.data_ptr()), ctypes.c_void_p(self._token_logit.data_ptr()),
                     ctypes.c_void_p(stream))
        return out, self._token

    def logits(self, hidden: torch.Tensor, chunk_rows: int = 4096) -> torch.Tensor:
        """The executor's ``logits`` (streamed_transformer_executor.py:177-209):
        float32 ``[vocab]`` on the host.  ``chunk_rows`` is accepted for the
        signature; the kernel streams the weight in one pass."""
        if int(chunk_rows) <= 0:
            raise ValueError("chunk_rows must be positive")
        out, _ = self.logits_device(hidden)
        return out.cpu()

    def greedy_token(self, hidden: torch.Tensor) -> int:
        """``int(argmax(nan_to_num(logits(hidden))))`` with the callers' constants."""
        _, token = self.logits_device(hidden)
        return int(token.item())
