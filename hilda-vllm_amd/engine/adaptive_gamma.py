"""Adaptive number of draft tokens, as in LLMEngine.step (llm_engine.py:197-208).

After every speculative step the step's acceptance rate (accepted draft tokens
over proposed draft tokens, summed over the sequences that took part) joins a
window of the last 20 steps. Once the window holds at least 5 rates, an average
above 0.8 raises gamma by one (up to 8) and an average below 0.4 lowers it by
one (down to 1). The window is not cleared when gamma changes.
"""
from __future__ import annotations


class AdaptiveGamma:

    def __init__(self, gamma: int, window: int = 20, min_samples: int = 5, raise_above: float = 0.8,
                 lower_below: float = 0.4, max_gamma: int = 8, min_gamma: int = 1):
        if not (min_gamma <= gamma <= max_gamma):
            raise ValueError(f"gamma {gamma} outside [{min_gamma}, {max_gamma}]")
        self.gamma = int(gamma)
        self.window = int(window)
        self.min_samples = int(min_samples)
        self.raise_above = float(raise_above)
        self.lower_below = float(lower_below)
        self.max_gamma = int(max_gamma)
        self.min_gamma = int(min_gamma)
        self.rates: list[float] = []

    def update(self, accepted: int, proposed: int) -> int:
        """Feeds one step's totals and returns gamma for the next step."""
        if proposed > 0:
            self.rates.append(accepted / proposed)
            if len(self.rates) > self.window:
                self.rates.pop(0)
            if len(self.rates) >= self.min_samples:
                avg = sum(self.rates) / len(self.rates)
                if avg > self.raise_above and self.gamma < self.max_gamma:
                    self.gamma += 1
                elif avg < self.lower_below and self.gamma > self.min_gamma:
                    self.gamma -= 1
        return self.gamma
