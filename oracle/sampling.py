"""Oracle of lm/sampling.py (test infrastructure, see oracle/__init__.py)."""
import torch


def next_token(logits: torch.Tensor, temperature: float, generator) -> int:
    """lm/sampling.py:4-10"""
    if temperature == 0.0:
        return int(torch.argmax(logits))
    probs = torch.softmax(logits.float() / temperature, dim=-1)
    return int(torch.multinomial(probs, 1, generator=generator))


def probabilities(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """lm/sampling.py:13-18"""
    if temperature == 0.0:
        return torch.nn.functional.one_hot(logits.argmax(dim=-1), logits.shape[-1]).float()
    return torch.softmax(logits.float() / temperature, dim=-1)
