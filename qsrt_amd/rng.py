"""Deterministic sign draws (mirrors ``qsrt/rng.py``).

``seeded_normal`` draws from a CPU ``torch.Generator`` and then moves the
result to ``device``.  The reference draws from a device-local generator
(``qsrt/rng.py:16-20``); a GPU stream would make the input/output signs -- and
therefore every payload -- depend on where the draw ran.  Drawing on the CPU
keeps the CPU oracle and the MI355X encoder on identical transforms; the CPU
stream equals ``manual_seed`` + ``randn`` (reference
``tests/test_qsrt_encoder.py:32-46``).
"""

from __future__ import annotations

import torch


def seeded_normal(length: int, *, device: torch.device | str, seed: int | None) -> torch.Tensor:
    generator = None
    if seed is not None:
        generator = torch.Generator(device="cpu")
        generator.manual_seed(int(seed))
    return torch.randn(length, generator=generator, dtype=torch.float32).to(device)
