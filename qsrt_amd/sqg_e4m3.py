"""SQG E4M3 reconstruction alphabets for the L16 trellis.

Mirrors the public surface of ``qsrt/sqg_e4m3.py`` in the reference.  Every
table here is host-side set-up (computed once, cached) that the HIP kernels
then consume as raw E4M3 bytes.

The trellis graph and its labels are separate objects: a codeword ``w`` (16
bits) is reached from state ``w >> K`` by branch ``w & (2^K - 1)``; the
label of ``w`` is an E4M3 byte.  The primary law ``sqg_xor_cheb_t12`` is

    rank(w)  = (stratum << (16 - K)) | phase          (a bijection of 2^16)
    label(w) = T12[rank(w) >> 4]                      (4 KiB modal staircase)

with ``phase``/``syndrome`` from a carry-mixed hash of the history and the
stratum a bit-reversed branch XOR syndrome
(reference ``qsrt/sqg_e4m3.py:259-301``).
"""

from __future__ import annotations

from functools import lru_cache

import torch

SQG_NORMAL_E4M3 = "sqg-normal-e4m3"
SQG_CHEB_NORMAL_E4M3 = "sqg-cheb-normal-e4m3"
SQG_XOR_CHEB_T12 = "sqg_xor_cheb_t12"

CODEWORDS = 1 << 16
# Tail clip and rational inverse-normal coefficients of the R44 control law
# (reference qsrt/sqg_e4m3.py:27-29).
_R44_CLIP = 1.0 / 2048.0
_R44_NUM = (1.25667142, 2.87422731, -9.02398882, 5.36810336, -0.46703015)
_R44_DEN = (1.0, 2.07630930, -8.08332684, 6.32135736, -1.31208298)


def _check_bits(bits: int, mode: str = "normal") -> None:
    if isinstance(bits, bool) or not isinstance(bits, int) or not 1 <= bits <= 6:
        raise ValueError("SQG supports integer K1 through K6")
    if mode != "normal":
        raise ValueError("the supported R44 mode is 'normal'")


def _bit_reverse(values: torch.Tensor, width: int) -> torch.Tensor:
    out = torch.zeros_like(values)
    for b in range(width):
        out |= ((values >> b) & 1) << (width - 1 - b)
    return out


def _split_codewords(bits: int) -> tuple[torch.Tensor, torch.Tensor, int]:
    words = torch.arange(CODEWORDS, dtype=torch.int64)
    return words >> bits, words & ((1 << bits) - 1), 16 - bits


# ---------------------------------------------------------------------------
# Primary law: carry-mixed rank map + modal T12 staircase
# ---------------------------------------------------------------------------


@lru_cache(maxsize=None)
def sqg_xor_rank_permutation(bits: int) -> torch.Tensor:
    """Rank of every codeword under the carry-mixed SQG map.

    Follows ``sqg_xor_rank_permutation`` (reference qsrt/sqg_e4m3.py:259-284):
    two triangular xorshifts over the ``16-K`` history bits, an odd affine
    multiply mod 2^32, low bits -> phase, top K bits -> syndrome.
    """

    _check_bits(bits)
    history, branch, width = _split_codewords(bits)
    hmask = (1 << width) - 1
    x = history ^ (history >> 11)
    x = x ^ ((x << 11) & hmask)
    p = (x * 0x3FA7D929 + 0xC928FD8E) & 0xFFFFFFFF
    stratum = _bit_reverse(branch, bits) ^ (p >> (32 - bits))
    return ((stratum << width) | (p & hmask)).contiguous()


def _e4m3_bytes(values: torch.Tensor) -> torch.Tensor:
    return values.float().to(torch.float8_e4m3fn).view(torch.uint8).contiguous()


def _finite_e4m3_rank_lut(values: torch.Tensor) -> torch.Tensor:
    """Round a monotone 65,536-entry rank law to canonical E4M3 bytes.

    Negative zero is folded to ``0x00`` so the byte contract is unique
    (reference qsrt/sqg_e4m3.py:196-213).
    """

    if values.ndim != 1 or values.numel() != CODEWORDS:
        raise ValueError("SQG rank-law values must contain exactly 65,536 entries")
    if not values.is_floating_point() or not bool(torch.isfinite(values).all()):
        raise ValueError("SQG rank-law values must be finite floating point")
    raw = _e4m3_bytes(values).clone()
    raw[(raw & 0x7F) == 0] = 0
    decoded = raw.view(torch.float8_e4m3fn).float()
    if not bool(torch.isfinite(decoded).all()):
        raise RuntimeError("SQG rank law rounded to a non-finite E4M3 value")
    if not bool((decoded[1:] >= decoded[:-1]).all()):
        raise RuntimeError("SQG rank law is not monotone after E4M3 rounding")
    return raw


@lru_cache(maxsize=1)
def sqg_cheb_normal_rank_e4m3_bytes() -> torch.Tensor:
    """Midpoint normal quantiles ``1.5 * ndtri((r + 0.5) / 2^16)`` as E4M3.

    Reference qsrt/sqg_e4m3.py:216-229 (float64 quantile, float32, then
    E4M3 round-to-nearest-even).
    """

    r = torch.arange(CODEWORDS, dtype=torch.float64)
    return _finite_e4m3_rank_lut(1.5 * torch.special.ndtri((r + 0.5) / CODEWORDS))


@lru_cache(maxsize=1)
def sqg_xor_cheb_t12_rank_lut_bytes() -> torch.Tensor:
    """4,096-byte modal staircase: the most frequent byte of each run of 16
    consecutive exact ranks, lowest byte value on ties
    (reference qsrt/sqg_e4m3.py:241-256)."""

    blocks = sqg_cheb_normal_rank_e4m3_bytes().reshape(4096, 16).to(torch.int64)
    counts = torch.zeros((4096, 256), dtype=torch.int64)
    counts.scatter_add_(1, blocks, torch.ones_like(blocks))
    top = counts.max(dim=1, keepdim=True).values
    # argmax over a 0/1 mask returns the first (lowest byte) maximiser.
    return (counts == top).to(torch.int8).argmax(dim=1).to(torch.uint8).contiguous()


@lru_cache(maxsize=None)
def _t12_labels(bits: int) -> torch.Tensor:
    return sqg_xor_cheb_t12_rank_lut_bytes()[sqg_xor_rank_permutation(bits) >> 4].contiguous()


def sqg_xor_cheb_t12_bytes(bits: int, *, device: torch.device | str = "cpu") -> torch.Tensor:
    """State-indexed E4M3 labels of the primary QSRT law (65,536 bytes)."""

    _check_bits(bits)
    return _t12_labels(bits).to(device=device).contiguous()


# ---------------------------------------------------------------------------
# Research-control laws (R44 rational compander, exact Chebyshev staircase)
# ---------------------------------------------------------------------------


def _mix(values: torch.Tensor, width: int, mults: tuple[int, int], shifts: tuple[int, int, int]) -> torch.Tensor:
    """Bijective xorshift-multiply mixer mod 2^width
    (reference qsrt/sqg_e4m3.py:39-60)."""

    mask = (1 << width) - 1

    def clamp(s: int) -> int:
        return min(max(s, 1), width - 1)

    x = values & mask
    for mult, shift in zip(mults, shifts[:2]):
        x = x ^ (x >> clamp(shift))
        x = (x * (mult | 1)) & mask
    x = x ^ (x >> clamp(shifts[2]))
    return x & mask


@lru_cache(maxsize=None)
def sqg_rank_permutation(bits: int) -> torch.Tensor:
    """Pre-projection rank of the R44 control graph
    (reference qsrt/sqg_e4m3.py:342-370)."""

    _check_bits(bits)
    history, branch, width = _split_codewords(bits)
    phase = _mix(history, width, (0x65AF, 0x16BF), (6, 4, 5))
    syndrome = _mix(history ^ 0x5105, width, (0x8693, 0x2A21), (2, 4, 4)) & ((1 << bits) - 1)
    stratum = (7 * (_bit_reverse(branch, bits) ^ syndrome)) & ((1 << bits) - 1)
    return ((stratum << width) | phase).contiguous()


def _r44_inverse_normal(p: torch.Tensor) -> torch.Tensor:
    a = 2.0 * p - 1.0
    x = a * a
    num = torch.full_like(x, _R44_NUM[-1])
    den = torch.full_like(x, _R44_DEN[-1])
    for c in reversed(_R44_NUM[:-1]):
        num = num * x + c
    for c in reversed(_R44_DEN[:-1]):
        den = den * x + c
    return a * num / den


@lru_cache(maxsize=None)
def _r44_bytes(bits: int) -> torch.Tensor:
    rank = sqg_rank_permutation(bits)
    p = ((rank.double() + 0.5) / CODEWORDS).clamp(_R44_CLIP, 1.0 - _R44_CLIP)
    values = (1.5 * _r44_inverse_normal(p)).float()
    if not bool(torch.isfinite(values).all()):
        raise RuntimeError("SQG compander produced a non-finite value")
    return _e4m3_bytes(values)


def sqg_e4m3_bytes(bits: int, mode: str, *, device: torch.device | str = "cpu") -> torch.Tensor:
    """R44 control labels (reference qsrt/sqg_e4m3.py:124-133)."""

    _check_bits(bits, mode)
    return _r44_bytes(bits).to(device=device).contiguous()


def sqg_e4m3_codebook(
    bits: int,
    mode: str,
    *,
    device: torch.device | str = "cpu",
    dtype: torch.dtype = torch.float16,
) -> torch.Tensor:
    if not dtype.is_floating_point:
        raise TypeError("SQG codebook dtype must be floating point")
    raw = sqg_e4m3_bytes(bits, mode, device=device)
    return raw.view(torch.float8_e4m3fn).to(dtype=dtype).contiguous()


def sqg_e4m3_bytes_from_rank_lut(
    bits: int, rank_lut: torch.Tensor, *, device: torch.device | str = "cpu"
) -> torch.Tensor:
    """Relabel the R44 graph with a rank-indexed E4M3 law
    (reference qsrt/sqg_e4m3.py:151-178)."""

    _check_bits(bits)
    if rank_lut.dtype != torch.uint8:
        raise TypeError("SQG rank LUT must contain raw uint8 E4M3 labels")
    if rank_lut.ndim != 1 or rank_lut.numel() != CODEWORDS:
        raise ValueError("SQG rank LUT must contain exactly 65,536 labels")
    rank_lut = rank_lut.detach().to("cpu").contiguous()
    if not bool(torch.isfinite(rank_lut.view(torch.float8_e4m3fn).float()).all()):
        raise ValueError("SQG rank LUT must contain only finite E4M3 labels")
    return rank_lut[sqg_rank_permutation(bits)].to(device=device).contiguous()


def sqg_e4m3_codebook_from_rank_lut(
    bits: int,
    rank_lut: torch.Tensor,
    *,
    device: torch.device | str = "cpu",
    dtype: torch.dtype = torch.float16,
) -> torch.Tensor:
    if not dtype.is_floating_point:
        raise TypeError("SQG codebook dtype must be floating point")
    raw = sqg_e4m3_bytes_from_rank_lut(bits, rank_lut, device=device)
    return raw.view(torch.float8_e4m3fn).to(dtype=dtype).contiguous()


@lru_cache(maxsize=None)
def sqg_cheb_normal_e4m3_bytes(bits: int) -> torch.Tensor:
    return sqg_e4m3_bytes_from_rank_lut(bits, sqg_cheb_normal_rank_e4m3_bytes()).contiguous()


# ---------------------------------------------------------------------------
# Named access
# ---------------------------------------------------------------------------


def sqg_codebook_bytes(
    bits: int,
    codebook: str,
    *,
    rate_axis: str | None = None,
    device: torch.device | str = "cpu",
) -> torch.Tensor:
    """State-indexed E4M3 labels of a named codebook
    (reference qsrt/sqg_e4m3.py:304-319)."""

    if codebook == SQG_XOR_CHEB_T12:
        return sqg_xor_cheb_t12_bytes(bits, device=device)
    if codebook == SQG_NORMAL_E4M3:
        return sqg_e4m3_bytes(bits, "normal", device=device)
    if codebook == SQG_CHEB_NORMAL_E4M3:
        return sqg_cheb_normal_e4m3_bytes(bits).to(device=device).contiguous()
    raise ValueError(f"unsupported SQG codebook: {codebook!r}")


def sqg_codebook(
    bits: int,
    codebook: str,
    *,
    rate_axis: str | None = None,
    device: torch.device | str = "cpu",
    dtype: torch.dtype = torch.float16,
) -> torch.Tensor:
    if not dtype.is_floating_point:
        raise TypeError("SQG codebook dtype must be floating point")
    raw = sqg_codebook_bytes(bits, codebook, rate_axis=rate_axis, device=device)
    return raw.view(torch.float8_e4m3fn).to(dtype=dtype).contiguous()
