"""The oracle's restatement of the reference sampler (oracle/text.py: SampleRawLogitsAdvanced and
sampleContinuation, internal/generate/sample.go:31-247) against the reference's own sampler test, the
draw's published test vectors and closed forms. The library's device sampler is checked against it on the
GPU (tests/test_gpu_sampling.py)."""
import math

import pytest

from oracle import text as T


def test_reference_sampler_cases():
    """TestSampleRawLogitsAdvanced (internal/generate/sample_test.go:15-42), for every draw."""
    logits = [2.0, 0.5, 5.0, -1.0]
    for u in (0.0, 0.3, 0.999999):
        assert T.sample_raw_logits(logits, [], 0.0, 1.0, 0, 1.0, u) == 2          # greedy
        assert T.sample_raw_logits(logits, [], 0.8, 1.0, 1, 1.0, u) == 2          # top-k 1
        assert T.sample_raw_logits([-10.0, -10.0, 20.0, -10.0], [], 1.0, 1.0, 0, 0.90, u) == 2  # top-p
        assert T.sample_raw_logits(logits, [2], 0.0, 10.0, 0, 1.0, u) != 2        # repetition penalty


def test_splitmix64_vectors():
    """The draw is SplitMix64's output stream (Vigna): seed 1234567 gives the published first outputs."""
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
            16408922859458223821]
    for k, w in enumerate(want):
        assert T.uniform_draw(1234567, k) == (w >> 11) * 2.0 ** -53
    assert 0.0 <= T.uniform_draw(0, 0) < 1.0


def test_inverse_cdf_closed_form():
    """Untruncated sampling inverts the softmax CDF: over a grid of draws, each token is chosen for a share
    of draws equal to its probability (to one grid step)."""
    logits = [0.3, -1.2, 2.0, 0.0, 1.1]
    N = 4000
    for temp in (0.5, 1.0, 2.0):
        counts = [0] * len(logits)
        for j in range(N):
            counts[T.sample_raw_logits(logits, [], temp, 1.0, 0, 1.0, (j + 0.5) / N)] += 1
        z = [math.exp(x / temp) for x in logits]
        for c, p in zip(counts, z):
            assert abs(c / N - p / sum(z)) <= 1.5 / N


def test_truncation_closed_forms():
    """top-k keeps the k most probable; top-p keeps the shortest prefix of the sorted probabilities whose
    sum reaches p; the draw is renormalised over what is kept."""
    logits = [math.log(x) for x in (0.1, 0.4, 0.2, 0.3)]   # probabilities 0.1 0.4 0.2 0.3 at T = 1
    picks = {T.sample_raw_logits(logits, [], 1.0, 1.0, 2, 1.0, (j + 0.5) / 100) for j in range(100)}
    assert picks == {1, 3}
    # top-p 0.65: 0.4 + 0.3 = 0.7 >= 0.65, kept {1, 3} renormalised to 4/7 and 3/7
    assert T.sample_raw_logits(logits, [], 1.0, 1.0, 0, 0.65, 0.57) == 1
    assert T.sample_raw_logits(logits, [], 1.0, 1.0, 0, 0.65, 0.58) == 3
    # top-p 0.3 keeps only the first: no draw can change it
    assert all(T.sample_raw_logits(logits, [], 1.0, 1.0, 0, 0.3, u) == 1 for u in (0.0, 0.5, 0.99))
    # a tie in probability orders by token id: with top-k 1, of two equal maxima the smaller id
    assert T.sample_raw_logits([1.0, 3.0, 3.0], [], 1.0, 1.0, 1, 1.0, 0.9) == 1


def test_repetition_penalty_rules():
    """sample.go:47-66: each distinct recent token once; positive logits divided, others multiplied."""
    # token 0 (logit 2) divided by 4 -> 0.5 < 1; token 1 (logit -1) multiplied -> -4
    assert T.sample_raw_logits([2.0, -1.0, 1.0], [0, 0, 1], 0.0, 4.0, 0, 1.0, 0.0) == 2
    # a repeated token is penalised once: 8 / 2 = 4 > 3 (twice would give 2 < 3)
    assert T.sample_raw_logits([8.0, 3.0], [0, 0], 0.0, 2.0, 0, 1.0, 0.0) == 0
    # out-of-range recent ids are skipped; a penalty of 1 changes nothing
    assert T.sample_raw_logits([1.0, 2.0], [7, -1], 0.0, 5.0, 0, 1.0, 0.0) == 1
    assert T.sample_raw_logits([2.0, 1.0], [0], 0.0, 1.0, 0, 1.0, 0.0) == 0


class _Fixed:
    """A session whose logits are a fixed table row per generated count."""

    def __init__(self, rows):
        self.rows, self.n = rows, 0

    def prefill(self, ids):
        return list(self.rows[0]) if ids else None

    def append(self, t):
        self.n += 1
        return list(self.rows[min(self.n, len(self.rows) - 1)])


def test_continuation_trigram_ban_and_window():
    """sampleContinuation (sample.go:196-247): after "a b" was followed by "c", a new "a b" cannot be
    followed by "c" again; the repetition window is the last 6 of prefix + reply; stops end the reply."""
    V = 6
    # greedy script a b c a b -> (c banned) -> next best
    rows = [[0, 0, 0, 0, 0, 0] for _ in range(7)]
    script = [1, 2, 3, 1, 2, 3, 4]
    for k, t in enumerate(script):
        rows[k][t] = 5.0
        rows[k][5] = 4.0
    got = T.sample_continuation(_Fixed(rows), [0], [], 7, 0.0, 1.0, 0, 1.0, seed=1)
    assert got[:5] == [1, 2, 3, 1, 2]
    assert got[5] == 5          # token 3 after "1 2" again is banned; the next highest is 5
    # stop token: the reply ends before it
    assert T.sample_continuation(_Fixed(rows), [0], [], 7, 0.0, 1.0, 0, 1.0, seed=1, stops=(3,)) == [1, 2]
    # the window reaches into the prompt prefix: the prompt's last token is penalised at step 0
    rows2 = [[0.0, 3.0, 2.9, 0, 0, 0]] * 3
    assert T.sample_continuation(_Fixed(rows2), [1], [1], 1, 0.0, 2.0, 0, 1.0, seed=1) == [2]
    assert T.sample_continuation(_Fixed(rows2), [1], [], 1, 0.0, 2.0, 0, 1.0, seed=1) == [1]
    # nothing from an empty context
    assert T.sample_continuation(_Fixed(rows2), [], [], 3, 1.0, 1.0, 0, 1.0, seed=1) == []
