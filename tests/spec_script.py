"""The reference's speculative-step test fixtures (crates/engine/src/spec/step.rs:466-910), restated:
the scripted verifier's rows, the plain loop, the scripted drafters and the speculative loop.

The rows are exact: each value is a 24-bit integer / 2^24 * 8 in f32, so every sampler sees the
same bits. The speculative loop verifies [x, d_1 .. d_k] in one call of a `verify(rows, drafts)`
that returns the picks it read (the accept loop of step.rs:340-385). The host cuts k so that the
loop never samples past its n tokens, which stands for `pick`'s `Next::End` at n (step.rs:881-888).
"""
VOCAB = 24  # step.rs:473
PROMPT = [3, 1, 4, 1, 5]  # step.rs:474
M64 = (1 << 64) - 1


def logits(history):
    """step.rs:478-493: a deterministic row from the history's last three tokens."""
    import numpy as np

    h = 0xCBF29CE484222325
    for t in history[max(0, len(history) - 3):]:
        h = ((h ^ t) * 0x00000100000001B3) & M64
    out = []
    for j in range(VOCAB):
        z = ((h ^ ((j * 0x9E3779B97F4A7C15) & M64)) + 0x9E3779B97F4A7C15) & M64
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        z ^= z >> 31
        out.append(np.float32(z >> 40) / np.float32(1 << 24) * np.float32(8.0))
    return np.array(out, dtype=np.float32)


class Plan:
    def __init__(self, length, wrong_at=None):
        self.length, self.wrong_at = length, wrong_at


class ScriptedDrafter:
    """step.rs:696-779: drafts the true stream by plan, one token replaced at `wrong_at`."""

    def __init__(self, truth, plans):
        self.truth, self.plans, self.seen, self.calls = list(truth), plans, 0, 0

    @classmethod
    def right(cls, truth):
        return cls(truth, [Plan(15)])

    @classmethod
    def wrong(cls, truth):
        return cls(truth, [Plan(15, 0)])

    @classmethod
    def half(cls, truth):
        return cls(truth, [Plan(15, 2)])

    @classmethod
    def none(cls, truth):
        return cls(truth, [Plan(0)])

    def draft(self, most):
        plan = self.plans[min(self.calls, len(self.plans) - 1)]
        self.calls += 1
        lo = min(self.seen, len(self.truth))
        hi = min(self.seen + min(plan.length, most), len(self.truth))
        d = self.truth[lo:hi]
        if plan.wrong_at is not None and plan.wrong_at < len(d):
            d[plan.wrong_at] = (d[plan.wrong_at] + 1) % VOCAB
        return d

    def observe(self, tokens):
        self.seen += len(tokens)


def plain(sampler, n):
    """step.rs:817-835: sample, emit, decode; the last token is never decoded. Returns (out, history)."""
    history = list(PROMPT)
    x = sampler.sample(logits(history))
    out = [x]
    while len(out) < n:
        history.append(x)
        x = sampler.sample(logits(history))
        out.append(x)
    return out, history


def speculate(sampler, drafter, n, most=4):
    """step.rs:837-906 with a fixed draft of up to `most` tokens (cfg(Some(4)), step.rs:794-807):
    k = 0 decodes and picks one row; otherwise rows i = 0..k are the rows after [x, d_1 .. d_i) and
    one verify call picks them. Returns (out, committed history, verify calls, drafts accepted)."""
    import numpy as np

    history = list(PROMPT)
    x = sampler.sample(logits(history))
    out = [x]
    drafter.observe(PROMPT)
    drafter.observe([x])
    calls = accepted = 0
    while len(out) < n:
        d = drafter.draft(most)[: n - len(out) - 1]
        if not d:
            history.append(x)
            y = sampler.sample(logits(history))
            out.append(y)
            drafter.observe([y])
            x = y
            continue
        tokens = [x] + d
        rows = np.stack([logits(history + tokens[: i + 1]) for i in range(len(d) + 1)])
        picks = sampler.verify(rows, d)
        calls += 1
        read = len(picks)
        accepted += read - 1
        out.extend(picks)
        drafter.observe(picks)
        history.extend(tokens[:read])
        x = picks[-1]
    return out, history, calls, accepted
