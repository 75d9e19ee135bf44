"""Seeded synthetic token streams for the drafter's benchmark workloads.

Every generator draws from ``numpy.random.default_rng(seed)`` (PCG64), so a
seed fixes the inputs bit for bit on any host.  Tokens are int32 >= 0.

Workloads (all shapes are the drafter's standard decode shapes):

* ``local_uniform``  -- B=8, S=2048, uniform vocab 32000, num_tokens in
  [512, 2048]; the row builder mixes fresh spans with copies of earlier spans.
* ``local_zipf``     -- B=64, S=8192, Zipf(1.1) over vocab 128256 (tokens are a
  seeded permutation of Zipf ranks), num_tokens in [2048, 8192], plus a
  [B, 17] sampled-token block carrying geometric(0.3) accepted tokens + 1.
* ``global_corpus``  -- 1024 sequences of 1k-8k tokens, 30% of each filled
  with whole copies of 64 shared template spans, the rest fresh Zipf
  segments; used to fill a 2^22-token corpus and a 2^16-token delta, with
  held-out sequences as the decode rows.

Nothing here touches a GPU; the arrays are plain numpy.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

VOCAB_SMALL = 32000
VOCAB_LARGE = 128256


class ZipfTokens:
    """Zipf(s) ranks over [1, V] by inverse CDF, mapped through a permutation."""

    def __init__(self, rng: np.random.Generator, vocab: int = VOCAB_LARGE,
                 s: float = 1.1):
        w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
        self.cdf = np.cumsum(w / w.sum())
        self.cdf[-1] = 1.0
        self.perm = rng.permutation(vocab).astype(np.int32)

    def draw(self, rng: np.random.Generator, n: int) -> np.ndarray:
        rank = np.searchsorted(self.cdf, rng.random(n), side="right")
        return self.perm[np.minimum(rank, self.perm.shape[0] - 1)]


def uniform_draw(vocab: int):
    def draw(rng: np.random.Generator, n: int) -> np.ndarray:
        return rng.integers(0, vocab, size=n, dtype=np.int64).astype(np.int32)
    return draw


def build_row(rng: np.random.Generator, length: int, draw) -> np.ndarray:
    """Copy-span / fresh-span mixture.

    Repeat until ``length`` tokens exist: with p=0.5 (always while the row is
    shorter than 16) append ``draw(U[8,64])`` fresh tokens, otherwise copy an
    earlier span of U[16,64] tokens (capped at the current length) from a
    uniform start.
    """
    out = np.empty(length + 64, dtype=np.int32)
    n = 0
    while n < length:
        if n < 16 or rng.random() < 0.5:
            seg = draw(rng, int(rng.integers(8, 65)))
            out[n:n + seg.shape[0]] = seg
            n += seg.shape[0]
        else:
            ln = min(int(rng.integers(16, 65)), n)
            st = int(rng.integers(0, n - ln + 1))
            out[n:n + ln] = out[st:st + ln]
            n += ln
    return out[:length].copy()


@dataclass
class DecodeBatch:
    """Token rows, committed counts and the next step's sampled block."""
    tokens: np.ndarray          # [B, S] int32
    num_tokens: np.ndarray      # [B] int32
    sampled: np.ndarray | None  # [B, T] int32, -1 padded
    meta: dict = field(default_factory=dict)


def _sampled_from_hidden(rng: np.random.Generator, hidden: np.ndarray,
                         num_tokens: np.ndarray, t: int) -> np.ndarray:
    """Row b carries min(geometric(0.3)-1, t-1)+1 tokens of its continuation."""
    b = hidden.shape[0]
    acc = np.minimum(rng.geometric(0.3, size=b) - 1, t - 1)
    sampled = np.full((b, t), -1, dtype=np.int32)
    for i in range(b):
        n = int(acc[i]) + 1
        st = int(num_tokens[i])
        seg = hidden[i, st:st + n]
        sampled[i, :seg.shape[0]] = seg
    return sampled


def local_uniform(seed: int = 1, b: int = 8, s: int = 2048,
                  lo: int = 512) -> DecodeBatch:
    rng = np.random.default_rng(seed)
    draw = uniform_draw(VOCAB_SMALL)
    tok = np.stack([build_row(rng, s, draw) for _ in range(b)])
    nt = rng.integers(lo, s, size=b, endpoint=True).astype(np.int32)
    return DecodeBatch(tok, nt, None, {"vocab": VOCAB_SMALL})


def local_zipf(seed: int = 2, b: int = 64, s: int = 8192, lo: int = 2048,
               t: int = 17) -> DecodeBatch:
    rng = np.random.default_rng(seed)
    z = ZipfTokens(rng)
    hidden = np.stack([build_row(rng, s + t, z.draw) for _ in range(b)])
    nt = rng.integers(lo, s, size=b, endpoint=True).astype(np.int32)
    sampled = _sampled_from_hidden(rng, hidden, nt, t)
    return DecodeBatch(hidden[:, :s].copy(), nt, sampled,
                       {"vocab": VOCAB_LARGE})


class TemplateCorpus:
    """Sequences sharing 64 template spans (30% of each sequence)."""

    def __init__(self, seed: int = 3, n_templates: int = 64,
                 frac: float = 0.3):
        self.rng = np.random.default_rng(seed)
        self.z = ZipfTokens(self.rng)
        self.frac = frac
        self.templates = [self.z.draw(self.rng, int(self.rng.integers(32, 257)))
                          for _ in range(n_templates)]

    def sequence(self, lo: int = 1024, hi: int = 8192) -> np.ndarray:
        rng = self.rng
        length = int(rng.integers(lo, hi, endpoint=True))
        budget = int(np.floor(self.frac * length))
        segs: list[np.ndarray] = []
        used = 0
        while used < budget:
            tpl = self.templates[int(rng.integers(0, len(self.templates)))]
            tpl = tpl[:budget - used]
            segs.append(tpl)
            used += tpl.shape[0]
        rest = length - used
        while rest > 0:
            seg = self.z.draw(rng, min(int(rng.integers(8, 65)), rest))
            segs.append(seg)
            rest -= seg.shape[0]
        order = rng.permutation(len(segs))
        return np.concatenate([segs[i] for i in order]).astype(np.int32)


@dataclass
class GlobalWorkload:
    active_docs: list[np.ndarray]   # docs resident in the corpus (oldest first)
    delta_docs: list[np.ndarray]    # docs appended to the delta after that
    batch: DecodeBatch              # decode rows drawn from held-out sequences


def global_corpus(seed: int = 3, capacity: int = 1 << 22,
                  delta_fill: int = 1 << 15, n_docs: int = 1024,
                  b: int = 64, s: int = 8192, t: int = 17,
                  seq_hi: int = 8192) -> GlobalWorkload:
    """Corpus docs (most recent that fit), delta docs, held-out decode rows.

    ``active_docs`` are the most recent of ``n_docs`` sequences whose total
    size including one separator each fits in ``capacity - 1`` (one slot is
    the sentinel).  ``delta_docs`` are further sequences appended while the
    running delta size (doc + separator) stays within ``delta_fill``.
    """
    tc = TemplateCorpus(seed)
    docs = [tc.sequence(hi=seq_hi) for _ in range(n_docs)]
    keep: list[np.ndarray] = []
    used = 0
    for d in reversed(docs):
        if used + d.shape[0] + 1 > capacity - 1:
            break
        keep.append(d)
        used += d.shape[0] + 1
    keep.reverse()
    delta: list[np.ndarray] = []
    dused = 0
    while True:
        d = tc.sequence(hi=min(seq_hi, max(1024, delta_fill // 4)))
        if dused + d.shape[0] + 1 > delta_fill:
            break
        delta.append(d)
        dused += d.shape[0] + 1
    rng = tc.rng
    rows = np.zeros((b, s), dtype=np.int32)
    nt = np.zeros(b, dtype=np.int32)
    sampled = np.full((b, t), -1, dtype=np.int32)
    for i in range(b):
        seq = tc.sequence(lo=1024 + t, hi=seq_hi + t)
        hi = min(seq.shape[0] - t, s)
        n = int(rng.integers(min(1024, hi), hi, endpoint=True))
        m = min(seq.shape[0], s)
        rows[i, :m] = seq[:m]
        nt[i] = n
        acc = min(int(rng.geometric(0.3)) - 1, t - 1) + 1
        seg = seq[n:n + acc]
        sampled[i, :seg.shape[0]] = seg
    return GlobalWorkload(keep, delta,
                          DecodeBatch(rows, nt, sampled, {"vocab": VOCAB_LARGE}))


@dataclass
class DecodeLoop:
    """A scripted decode loop: initial rows, per-step sampled blocks and the
    harvests (every ``every`` steps the ``harvest`` longest rows, ties to
    the lower index, are harvested at their host-mirrored lengths and reset
    to fresh prefixes)."""
    tokens: np.ndarray              # [B, S] int32 initial rows
    num_tokens: np.ndarray          # [B] int32
    sampled: np.ndarray             # [steps, B, T] int32, -1 padded
    harvests: dict                  # step -> (rows, lengths, new rows, new counts)


def decode_loop(seed: int = 5, b: int = 256, s: int = 16384,
                steps: int = 1000, t: int = 17, every: int = 64,
                harvest: int = 16, lo: int = 2048, hi: int = 8192
                ) -> DecodeLoop:
    """Config-2-style rows (Zipf tokens, copy/fresh spans) whose every step
    accepts min(geometric(0.3) - 1, T - 1) + 1 tokens of the row's own
    hidden continuation; the host mirrors each row's count exactly as
    update_state advances it (base + accepted, not clipped)."""
    rng = np.random.default_rng(seed)
    z = ZipfTokens(rng)
    hidden = np.stack([build_row(rng, s + t, z.draw) for _ in range(b)])
    q = rng.integers(lo, hi, size=b, endpoint=True).astype(np.int64)
    tokens = hidden[:, :s].copy()
    num_tokens = q.astype(np.int32)
    sampled = np.full((steps, b, t), -1, dtype=np.int32)
    harvests = {}
    for i in range(steps):
        acc = np.minimum(rng.geometric(0.3, size=b) - 1, t - 1) + 1
        for r in range(b):
            n = int(acc[r])
            st = int(q[r])
            seg = hidden[r, st:st + n] if st < hidden.shape[1] else hidden[r, :0]
            if seg.shape[0] < n:
                seg = np.concatenate([seg, z.draw(rng, n - seg.shape[0])])
            sampled[i, r, :n] = seg
        q += acc
        if (i + 1) % every == 0:
            order = np.lexsort((np.arange(b), -q))[:harvest]
            rows = [int(r) for r in order]
            lengths = [int(min(q[r], s)) for r in rows]
            new_rows = np.stack([build_row(rng, s + t, z.draw) for _ in rows])
            new_q = rng.integers(lo, hi, size=len(rows), endpoint=True)
            for j, r in enumerate(rows):
                hidden[r] = new_rows[j]
                q[r] = new_q[j]
            harvests[i] = (rows, lengths, new_rows[:, :s].copy(),
                           new_q.astype(np.int32))
    return DecodeLoop(tokens, num_tokens, sampled, harvests)
