"""The per-block work of a batched BlockLDLQ traversal on the GPU.

One 16-row step of ``ldlq`` / ``ldlq_mixed_batched`` (reference
``qsrt/exl3_encoder_backend.py:420-539``, ``:1190-1478``) around the tile
Viterbi is two launches for the whole batch (``include/qsrt_amd.h``):
``qsrt_ldlq_targets`` writes every member's feedback targets straight into
their slots of the rate-grouped tile buffer, and ``qsrt_ldlq_commit`` writes
the reconstruction and states back.  The product-cache update after each
span stays a matrix-core product per member (``qsrt_amd.gemm``).

Precision: the regularised weight, the factor and the product cache are
float64 and the reconstruction FP32 (its labels are exact); each target is
its float64 sum rounded once to FP32, the contract of the float64 CPU
recursion the payloads are compared with.
"""

from __future__ import annotations

import torch

from . import _native


class LdlqStep:
    """Device views of one traversal: float64 sources ``weights [S, K, N]``
    and ``Ls [S, K, K]``; per member float32 ``weights_q``, float64
    ``prod_cache [B, K, N]`` and ``encoded [B, K/16, N/16, 256]``; member
    ``m`` reads source ``src[m]`` and scales its feedback by
    ``multipliers[m]``."""

    def __init__(self, weights, Ls, weights_q, prod_cache, encoded, src, multipliers):
        S, K, N = weights.shape
        B = weights_q.shape[0]
        for name, t, shape, dtype in (("weights", weights, (S, K, N), torch.float64),
                                      ("Ls", Ls, (S, K, K), torch.float64),
                                      ("weights_q", weights_q, (B, K, N), torch.float32),
                                      ("prod_cache", prod_cache, (B, K, N), torch.float64),
                                      ("encoded", encoded, (B, K // 16, N // 16, 256), torch.int16)):
            if tuple(t.shape) != shape or t.dtype != dtype or not t.is_contiguous() or not t.is_cuda:
                raise ValueError(f"LDLQ step: {name} must be a contiguous {dtype} CUDA tensor of shape {shape}")
        if K % 16 or N % 16:
            raise ValueError("LDLQ step: K and N must be multiples of 16")
        src = list(range(B)) if src is None else [int(s) for s in src]
        if len(src) != B or any(not 0 <= s < S for s in src):
            raise ValueError("LDLQ step: one source index in range per member")
        if len(multipliers) != B:
            raise ValueError("LDLQ step: one feedback multiplier per member")
        dev = weights.device
        self.W, self.L, self.Q, self.P, self.E = weights, Ls, weights_q, prod_cache, encoded
        self.B, self.K, self.N = B, K, N
        self.src = torch.tensor(src, dtype=torch.int32, device=dev)
        self.mult = torch.tensor([float(m) for m in multipliers], dtype=torch.float64, device=dev)
        self._stream = lambda: _native.stream_handle(dev)

    @property
    def tiles(self) -> int:
        return self.B * (self.N // 16)

    def _check_slot(self, slot: torch.Tensor) -> None:
        if slot.dtype != torch.int32 or slot.numel() != self.tiles or not slot.is_contiguous():
            raise ValueError("LDLQ step: slot must be contiguous int32 [B * N / 16]")

    def targets(self, tiles: torch.Tensor, slot: torch.Tensor, blk: int, end: int) -> None:
        """Targets of rows [blk, blk + 16) of a span ending at ``end`` into
        ``tiles [B * N / 16, 256]`` at ``slot`` (a permutation of the tiles)."""

        self._check_slot(slot)
        if tiles.shape != (self.tiles, 256) or tiles.dtype != torch.float32 or not tiles.is_contiguous():
            raise ValueError("LDLQ step: tiles must be contiguous float32 [B * N / 16, 256]")
        K, N = self.K, self.N
        _native.check(_native.lib().qsrt_ldlq_targets(
            tiles.data_ptr(), self.W.data_ptr(), self.L.data_ptr(), self.Q.data_ptr(), self.P.data_ptr(),
            self.src.data_ptr(), self.mult.data_ptr(), slot.data_ptr(), self.B, K, N, K * N, K * K, K * N, K * N,
            int(blk), int(end), self._stream()), "qsrt_ldlq_targets")

    def commit(self, recon: torch.Tensor, states: torch.Tensor, slot: torch.Tensor, blk: int) -> None:
        """Reconstruction and states of rows [blk, blk + 16) from the tile
        buffers (tile ``slot[m N/16 + t]`` is member m's column tile t)."""

        self._check_slot(slot)
        if (recon.shape != (self.tiles, 256) or recon.dtype != torch.float32 or not recon.is_contiguous()
                or states.shape != (self.tiles, 256) or states.dtype != torch.int16 or not states.is_contiguous()):
            raise ValueError("LDLQ step: recon / states must be contiguous [B * N / 16, 256] float32 / int16")
        K, N = self.K, self.N
        _native.check(_native.lib().qsrt_ldlq_commit(
            self.Q.data_ptr(), self.E.data_ptr(), recon.data_ptr(), states.data_ptr(), slot.data_ptr(), self.B, K,
            N, K * N, (K // 16) * (N // 16) * 256, int(blk), self._stream()), "qsrt_ldlq_commit")
