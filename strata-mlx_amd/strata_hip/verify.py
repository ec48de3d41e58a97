"""The draft-verify step: one pass of the trunk over the window [next token, *guesses], the trunk's own token after
each row, the longest run of guesses it agrees with, and the commit that keeps only those positions in the paged
caches — strata_mlx/engine.py:710-749 (`Engine.step`) and 372-376 (`_commit`'s attention part, `cache.trim`).

The trunk pass is the caller's `forward(window) -> logits (T, vocab)`: the decode layers built from this package
(Attention over a PagedKVCache, the MoE block, the dense layers), which append the window's T positions to every
cache. `choose(logits, window)` picks the trunk's token after each row (greedy by default, as the engine's greedy
sampling does, sampler.py:77-78). What a drafter proposes next is the caller's: `guesses` is set between steps.
The reference's n-gram lookup, guess policy and timing stats are not part of the path.
"""

from dataclasses import dataclass, field

import torch

MAX_WINDOW = 8  # strata_mlx/drafting.py:25: the widest verify window


@dataclass
class Stats:
    """strata_mlx/engine.py:132-138 (without the lookup's count): passes, tokens settled, guesses sent, guesses the
    trunk agreed with, and how many passes kept 0, 1, ... guesses."""

    steps: int = 0
    tokens: int = 0
    drafted: int = 0
    accepted: int = 0
    by_position: list = field(default_factory=lambda: [0] * MAX_WINDOW)


def kept_of(window: list, choice: list, stop: tuple = ()) -> int:
    """How many guesses the trunk keeps (engine.py:727-729): guess t + 1 stays while the trunk's token after row t
    is that guess and is not a stop token."""
    kept = 0
    while kept < len(window) - 1 and window[kept + 1] == choice[kept] and choice[kept] not in stop:
        kept += 1
    return kept


def greedy(logits: torch.Tensor, window: list) -> list:
    """The trunk's token after each row: the largest logit, the lowest index among equals (one sync for the
    window)."""
    if logits.shape[0] != len(window):
        raise ValueError(f"logits of {logits.shape[0]} rows for a window of {len(window)}")
    return torch.argmax(logits.float(), dim=-1).tolist()


class Verifier:
    """`Engine.step` over caches that hold the conversation: `next_token` (the settled token not yet read) and
    `guesses` (the drafter's, at most MAX_WINDOW - 1 used) go in, the settled tokens come out, the caches keep
    exactly the positions of the tokens read."""

    def __init__(self, forward, caches, choose=greedy):
        self.forward, self.caches, self.choose = forward, list(caches), choose
        self.next_token = None
        self.guesses = []
        self.tokens = []  # the tokens the caches hold, in order
        self.stats = Stats()

    def commit(self, window: list, n: int):
        """Keep the first n tokens of the window (engine.py:372-376): every cache drops the rest."""
        T = len(window)
        if not 1 <= n <= T:
            raise ValueError(f"keep {n} of a window of {T}")
        for cache in self.caches:
            cache.trim(T - n)
        self.tokens += window[:n]

    def step(self, limit: int = MAX_WINDOW, stop: tuple = ()) -> list:
        """One pass of the trunk (engine.py:710-749). Returns the tokens it settled, the last of which is not read
        yet; at most `limit`, nothing after a token in `stop`."""
        if self.next_token is None:
            raise ValueError("step: no token to read (read a prompt first)")
        window = [self.next_token, *self.guesses[: MAX_WINDOW - 1]][: max(1, limit)]
        T = len(window)
        logits = self.forward(window)
        choice = self.choose(logits, window)
        kept = kept_of(window, choice, stop)
        n = kept + 1
        self.commit(window, n)
        settled = choice[:n]
        self.next_token = settled[-1]
        self.guesses = []
        s = self.stats
        s.steps, s.tokens, s.drafted, s.accepted = s.steps + 1, s.tokens + n, s.drafted + T - 1, s.accepted + kept
        s.by_position[kept] += 1
        return settled
