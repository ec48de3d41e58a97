"""The draft-verify step (strata_hip.verify, engine.py:710-749) on the CPU, with a toy trunk whose next token depends
on the whole history its caches hold: whatever the guesses (right, wrong, too many, past a stop token), the settled
tokens are the ones one-token-at-a-time greedy decoding gives, the caches hold exactly the tokens read, and the
statistics count what was sent and kept."""

import numpy as np
import pytest
import torch

from strata_hip import verify as SV

V = 61  # vocab


def next_of(history: list) -> int:
    """The toy trunk's greedy token after `history` (every token of it matters)."""
    h = 7
    for t in history:
        h = (h * 31 + t) % 1_000_003
    return h % V


class ToyCache:
    """Holds tokens as a paged cache holds positions: forward appends, trim drops from the end."""

    def __init__(self):
        self.tokens = []

    def trim(self, n: int) -> int:
        n = min(n, len(self.tokens))
        del self.tokens[len(self.tokens) - n:]
        return n


def toy_trunk(caches):
    def forward(window):
        base = list(caches[0].tokens)
        for c in caches:
            assert c.tokens == base  # every layer's cache holds the same positions
            c.tokens += window
        logits = torch.full((len(window), V), -1.0)
        for t in range(len(window)):
            logits[t, next_of(base + window[: t + 1])] = 1.0
        return logits
    return forward


def reference_decode(prompt: list, n: int, stop=()) -> list:
    """One token a pass, no guesses."""
    out, hist = [], list(prompt)
    tok = next_of(hist)
    out.append(tok)
    while len(out) < n and tok not in stop:
        hist.append(tok)
        tok = next_of(hist)
        out.append(tok)
    return out


def start(prompt, n_caches=3):
    caches = [ToyCache() for _ in range(n_caches)]
    for c in caches:
        c.tokens += prompt
    v = SV.Verifier(toy_trunk(caches), caches)
    v.tokens = list(prompt)
    v.next_token = next_of(prompt)
    return v, caches


def run(v, caches, n, drafter, stop=()):
    out = [v.next_token]
    while len(out) < n and out[-1] not in stop:
        v.guesses = drafter(v.tokens + [v.next_token])
        settled = v.step(n - len(out), stop)
        out += settled
        for c in caches:
            assert c.tokens == v.tokens  # the caches hold exactly the tokens read
        assert v.tokens[-1] != v.next_token or len(settled) >= 1
    return out


@pytest.mark.parametrize("seed", range(6))
def test_guesses_never_change_the_answer(seed):
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, V, 5).tolist()
    want = reference_decode(prompt, 40)

    def drafter(history):  # the true continuation, with some guesses made wrong
        g, h = [], list(history)
        for _ in range(int(rng.integers(0, 10))):
            t = next_of(h)
            if rng.random() < 0.25:
                t = (t + 1 + int(rng.integers(0, V - 1))) % V
            g.append(t)
            h.append(t)
        return g

    v, caches = start(prompt)
    got = run(v, caches, 40, drafter)
    assert got[:40] == want
    s = v.stats
    assert s.tokens == len(v.tokens) - len(prompt)
    assert s.accepted <= s.drafted and sum(s.by_position) == s.steps
    assert s.tokens == s.steps + s.accepted  # a pass settles its kept guesses and one token of its own


def test_right_guesses_settle_a_window_a_pass():
    prompt = [3, 1, 4, 1, 5]
    want = reference_decode(prompt, 33)

    def oracle(history):
        g, h = [], list(history)
        for _ in range(SV.MAX_WINDOW - 1):
            h.append(next_of(h))
            g.append(h[-1])
        return g

    v, caches = start(prompt)
    got = run(v, caches, 33, oracle)
    assert got == want
    assert v.stats.steps == 4 and v.stats.by_position[SV.MAX_WINDOW - 1] == 4  # 1 + 4 x 8 tokens


def test_wrong_guesses_are_trimmed_and_cost_nothing_but_the_pass():
    prompt = [9, 9, 9]
    want = reference_decode(prompt, 12)
    v, caches = start(prompt)
    got = run(v, caches, 12, lambda h: [(next_of(h) + 1) % V] * 5)
    assert got == want
    assert v.stats.accepted == 0 and v.stats.by_position[0] == v.stats.steps == 11


def test_a_stop_token_ends_the_run_and_the_limit_caps_the_window():
    prompt = [1, 2, 3, 4]
    seq = reference_decode(prompt, 30)
    stop = (seq[5],)
    want = reference_decode(prompt, 30, stop)
    assert want[-1] == seq[5] and len(want) == 6

    def oracle(history):
        g, h = [], list(history)
        for _ in range(7):
            h.append(next_of(h))
            g.append(h[-1])
        return g

    v, caches = start(prompt)
    windows = []
    fwd = v.forward
    v.forward = lambda w: (windows.append(len(w)), fwd(w))[1]
    got = run(v, caches, 30, oracle, stop)
    assert got == want  # nothing settled after the stop token
    assert windows and max(windows) <= SV.MAX_WINDOW
    v2, caches2 = start(prompt)
    v2.guesses = oracle(v2.tokens + [v2.next_token])
    assert len(v2.step(limit=3)) == 3 and len(v2.tokens) == len(prompt) + 3


def test_kept_of_follows_the_reference_rule():
    assert SV.kept_of([5], []) == 0
    assert SV.kept_of([5, 6, 7, 8], [6, 7, 8, 9]) == 3
    assert SV.kept_of([5, 6, 7, 8], [6, 0, 8, 9]) == 1
    assert SV.kept_of([5, 6, 7, 8], [1, 7, 8, 9]) == 0
    assert SV.kept_of([5, 6, 7, 8], [6, 7, 8, 9], stop=(7,)) == 1  # the guess after a stop token is not kept
    with pytest.raises(ValueError):
        SV.greedy(torch.zeros(3, 4), [1, 2])
    assert SV.greedy(torch.tensor([[0.0, 2.0, 2.0], [5.0, 1.0, 5.0]]), [1, 2]) == [1, 0]  # ties to the lower index
