"""JevstralDecider's token loop (src/Jevstral/JevstralDecider.cs:246-354) over libjev.

`TreeDecider.decide` takes what DecideAsync has after tokenizing (the prompt's
prefix tokens, the tokens of the same question over empty data, and one
branch of tokens per option) and does what DecideAsync does with them:

* reuse the cache: keep the leading tokens this prefix shares with the
  previous call's trunk (truncate), or restore the longest remembered question
  prefix (the snapshot LRU), or the system-prompt snapshot, or start cold --
  in the reference's order of preference (JevstralDecider.cs:255-286);
* one tree pass: the rest of the prefix as the trunk, every option's query as
  a branch, only the verdict rows of the LM head;
* leave the cache holding the whole prefix, remember this question's prefix;
* margins z_i = max(yes rows) - max(no rows), p = softmax(z / T).

Every kernel is batch-invariant, so a warm call returns the same bits as a
cold one.  Prompt rendering and tokenization are not part of this library.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import _lib as L
from .model import margins as _margins
from .prefix_cache import SystemPromptCache


def common_prefix(a: Sequence[int], b: Sequence[int]) -> int:
    """CommonPrefix (JevstralDecider.cs:356-361)."""
    x = np.asarray(a, dtype=np.int64).ravel()
    y = np.asarray(b, dtype=np.int64).ravel()
    n = min(x.size, y.size)
    diff = np.nonzero(x[:n] != y[:n])[0]
    return int(diff[0]) if diff.size else n


def temperature_for(question_type: str, n_options: int, table: Optional[Dict[str, float]] = None) -> float:
    """TemperatureFor (JevstralDecider.cs:320-328): the "type:bucket" key wins
    over "type"; a missing key means 1; never below 1e-3."""
    if question_type not in ("noul", "choice", "score"):
        question_type = "choice"
    k = n_options
    bucket = "2" if k <= 2 else "3-5" if k <= 5 else "6-10" if k <= 10 else "11+"
    table = table or {}
    for key in (f"{question_type}:{bucket}", question_type):
        if key in table:
            return max(float(table[key]), 1e-3)
    return 1.0


@dataclass
class DecisionResult:
    """DecisionResult (JevstralDecider.cs:63-84) without the labels."""
    probabilities: np.ndarray
    margins: np.ndarray
    prefix_tokens: int
    suffix_tokens: int
    cached_tokens: int = 0

    @property
    def best(self) -> int:
        """Index of the most probable option (Kernels.ArgMax: the first maximum)."""
        from .reasoning import index_of_max
        return index_of_max(self.probabilities)


@dataclass
class _QuestionSnapshot:
    tokens: np.ndarray
    state: object  # a DeviceSnapshot (HBM) when the model offers one, else the flat host array


class TreeDecider:
    """One decider owns one model's KV cache; not thread-safe."""

    def __init__(self, model, yes_rows: Sequence[int], no_rows: Sequence[int],
                 system_tokens: Optional[Sequence[int]] = None, question_cache_size: int = 8):
        self.model = model
        self._yes = [int(r) for r in yes_rows]
        self._no = [int(r) for r in no_rows]
        if not self._yes or not self._no:
            raise L.DataError(L.JEV_EDATA, "The model's vocabulary has no 'yes'/'no' tokens; this does not look "
                                           "like a Shieldstral checkpoint.")
        self._rows = self._yes + self._no
        # OpenAsync (JevstralDecider.cs:175-193): the system block is captured once
        self._system: Optional[SystemPromptCache] = None
        self._resident = np.zeros(0, np.int32)
        if system_tokens is not None:
            self._system = SystemPromptCache.capture(model, system_tokens)
            self._resident = self._system.tokens.copy()
        self._questions: List[_QuestionSnapshot] = []  # most recent last
        self._question_hits = 0
        self.question_cache_size = question_cache_size

    @property
    def question_cache_hits(self) -> int:
        """Calls whose question prefix came from a snapshot rather than the resident trunk."""
        return self._question_hits

    @property
    def system_tokens(self) -> int:
        return self._system.token_count if self._system is not None else 0

    def decide(self, prefix: Sequence[int], question_tokens: Sequence[int], branches: Sequence[Sequence[int]],
               temperature: float = 1.0) -> DecisionResult:
        """DecideAsync (JevstralDecider.cs:246-318) after tokenization.

        `question_tokens` is the prompt rendered for the same question with an
        empty state; its common prefix with `prefix` is the question part that
        the snapshot LRU keeps."""
        if len(branches) < 2:
            raise L.ArgumentError(L.JEV_EINVAL, "A decision needs at least two options.")
        prefix = np.ascontiguousarray(np.asarray(prefix, dtype=np.int32).ravel())
        m = self.model
        start = common_prefix(prefix, self._resident)
        question_length = common_prefix(prefix, question_tokens)
        snapshot = self._find_snapshot(prefix, start) if start < question_length else None
        if snapshot is not None:
            m.kv_restore(snapshot.state, len(snapshot.tokens))  # a copy inside HBM for a device snapshot
            start = len(snapshot.tokens)
            self._question_hits += 1
        elif start > 0 and start >= self.system_tokens:
            m.kv_truncate(start)
        elif self._system is not None and self._system.is_prefix_of(prefix):
            self._system.restore_into(m)
            start = self._system.token_count
        else:
            m.reset_kv_cache()
            start = 0
        # never an empty trunk: re-run the prefix's last token so the branches
        # follow a token computed in this pass's layout
        if start == len(prefix):
            start -= 1
            m.kv_truncate(start)

        suffix_tokens = sum(len(b) for b in branches)
        verdicts = m.forward_tree(prefix[start:], branches, self._rows)
        m.kv_truncate(len(prefix))
        self._resident = prefix
        self._remember(prefix, question_length)

        z, p = _margins(np.stack(verdicts), len(self._yes), len(self._no), temperature)
        return DecisionResult(p, z, len(prefix), suffix_tokens, cached_tokens=start)

    def _find_snapshot(self, prefix: np.ndarray, at_least: int) -> Optional[_QuestionSnapshot]:
        """FindSnapshot (JevstralDecider.cs:330-345): the longest remembered
        question prefix beyond `at_least` that `prefix` starts with; moved to
        the most-recent end."""
        best = None
        for q in self._questions:
            n = len(q.tokens)
            if at_least < n <= len(prefix) and common_prefix(prefix, q.tokens) == n \
                    and (best is None or n > len(best.tokens)):
                best = q
        if best is not None:
            self._questions.remove(best)
            self._questions.append(best)
        return best

    def _remember(self, prefix: np.ndarray, question_length: int) -> None:
        """Remember (JevstralDecider.cs:348-354): snapshot this call's question
        prefix unless it is already kept; oldest evicted first."""
        if self.question_cache_size <= 0 or question_length <= self.system_tokens:
            return
        for q in self._questions:
            if len(q.tokens) == question_length and common_prefix(prefix, q.tokens) == question_length:
                return
        take = getattr(self.model, "kv_snapshot_device", None) or self.model.kv_snapshot
        self._questions.append(_QuestionSnapshot(prefix[:question_length].copy(), take(question_length)))
        while len(self._questions) > self.question_cache_size:
            evicted = self._questions.pop(0)
            if hasattr(evicted.state, "close"):
                evicted.state.close()
