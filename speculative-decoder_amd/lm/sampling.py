"""Temperature sampling helpers (reference: lm/sampling.py:4-18).

`probabilities` runs the softmax / one-hot kernel of libspecdec.so.
"""
from __future__ import annotations

import torch

from specdec import ops


def next_token(logits: torch.Tensor, temperature: float, generator: torch.Generator | None) -> int:
    """logits: [V].  Temperature 0 is greedy (the first maximum wins, so ties go
    to the lower id); otherwise one multinomial draw from the softmax with
    `generator` (on the generator's device)."""
    if temperature == 0.0:
        return int(torch.argmax(logits))
    probs = probabilities(logits, temperature)
    dev = generator.device if generator is not None else torch.device("cpu")
    return int(torch.multinomial(probs.to(dev), 1, generator=generator))


def probabilities(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """[..., V] logits -> float32 probabilities on the logits' GPU.  Temperature
    0 gives the one-hot of the argmax (lowest id among ties), which turns
    accept-reject into exact greedy verification."""
    if logits.device.type != "cuda":
        logits = logits.to("cuda")
    return ops.probabilities(logits, temperature)
