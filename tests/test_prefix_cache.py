"""Prefix snapshots and the decider's cache reuse on the host (no GPU).

SystemPromptCache (SystemPromptCache.cs): the SHKV bytes are checked field by
field against BinaryWriter's encoding written out here independently (7-bit
length prefixes as closed forms), the fingerprint against its documented
string, and TryLoad's misses one by one.

TreeDecider (JevstralDecider.cs:246-354) runs over a stand-in model whose
"KV cache" is the list of tokens in its slots and whose verdict logits are a
hash of exactly what each branch sees.  A warm decider must therefore reach
the same logical context -- and the same margins -- as a cold one, while
reusing what DecideAsync reuses (DeciderTests.cs:99-138 on real weights; the
bitwise version runs on the GPU in test_gpu_prefix_cache.py).
"""
import hashlib
import io
import os
import struct
from dataclasses import dataclass

import numpy as np
import pytest

import jev
from jev import prefix_cache as P


@dataclass
class _Cfg:
    n_layers: int = 2
    n_kv_heads: int = 1
    head_dim: int = 4
    architecture: str = "mistral3"


class FakeModel:
    """KV cache = the token in each slot; snapshots carry the tokens in
    KvCache.Snapshot's element count (2 * layers * kv heads * length * 128)."""

    def __init__(self, path=None):
        self.config = _Cfg()
        self.model_path = path
        self.cache = []
        self.ops = []

    @property
    def cached_token_count(self):
        return len(self.cache)

    def _per_token(self):
        c = self.config
        return 2 * c.n_layers * c.n_kv_heads * c.head_dim

    def reset_kv_cache(self):
        self.ops.append(("reset",))
        self.cache = []

    def prefill(self, tokens):
        self.ops.append(("prefill", len(tokens)))
        self.cache += [int(t) for t in tokens]

    def kv_truncate(self, n):
        self.ops.append(("truncate", n))
        if n < 0 or n > len(self.cache):
            raise jev.ArgumentError(1, "bad length")
        self.cache = self.cache[:n]

    def kv_snapshot(self, n):
        self.ops.append(("snapshot", n))
        return np.repeat(np.asarray(self.cache[:n], np.float32), self._per_token())

    def kv_restore(self, state, n):
        self.ops.append(("restore", n))
        assert state.size == n * self._per_token()
        self.cache = [int(v) for v in np.asarray(state).reshape(n, -1)[:, 0]]

    def forward_tree(self, trunk, branches, rows):
        self.ops.append(("tree", len(trunk)))
        ctx = self.cache + [int(t) for t in trunk]
        out = []
        for b in branches:
            seen = tuple(ctx + [int(t) for t in b])
            seed = int.from_bytes(hashlib.sha256(repr(seen).encode()).digest()[:8], "little")
            out.append(np.random.default_rng(seed).standard_normal(len(rows)).astype(np.float32))
        self.cache = ctx + [int(t) for b in branches for t in b]
        return out


# ------------------------------------------------------------------ SHKV bytes

@pytest.mark.parametrize("n,prefix", [(0, b"\x00"), (1, b"\x01"), (127, b"\x7f"), (128, b"\x80\x01"),
                                      (300, b"\xac\x02"), (16383, b"\xff\x7f"), (16384, b"\x80\x80\x01")])
def test_binarywriter_string_length_prefix(n, prefix):
    s = "a" * n
    enc = P.encode_dotnet_string(s)
    assert enc == prefix + s.encode()
    assert P._read_dotnet_string(io.BytesIO(enc)) == s


def test_binarywriter_string_counts_utf8_bytes():
    assert P.encode_dotnet_string("é") == b"\x02\xc3\xa9"


def test_shkv_layout_field_by_field():
    fp = "0123456789abcdef" * 4
    c = jev.SystemPromptCache([5, 7, 300], np.array([1.5, -2.0, 0.0, 3.25, 7.0, -0.5], np.float32), fp)
    b = c.to_bytes()
    assert b[:4] == b"VKHS"  # 0x53484B56 little-endian
    assert struct.unpack_from("<i", b, 4)[0] == 1
    assert b[8] == 64 and b[9:73] == fp.encode()
    assert struct.unpack_from("<i", b, 73)[0] == 3
    assert struct.unpack_from("<3i", b, 77) == (5, 7, 300)
    assert struct.unpack_from("<q", b, 89)[0] == 6
    assert struct.unpack_from("<6f", b, 97) == (1.5, -2.0, 0.0, 3.25, 7.0, -0.5)
    assert len(b) == 97 + 24
    assert c.byte_size == 24 and c.token_count == 3


# ------------------------------------------------------------------ fingerprint

def _sha(text):
    return hashlib.sha256(text.encode("utf-8")).hexdigest()


def test_fingerprint_is_the_documented_string(tmp_path):
    f = tmp_path / "model.gguf"
    f.write_bytes(b"x" * 1234)
    ns = 1_700_000_000_123_456_789
    os.utime(f, ns=(ns, ns))
    m = FakeModel(str(f))
    ticks = 621355968000000000 + ns // 100  # DateTime ticks of the write time
    assert P.fingerprint(m, [5, 7, 300]) == _sha(f"model.gguf|1234|{ticks}|mistral3|2x1x4|3:5,7,300,")
    assert P.fingerprint(FakeModel(str(tmp_path / "gone.gguf")), [1]) == _sha("gone.gguf|-1|-1|mistral3|2x1x4|1:1,")
    assert P.fingerprint(FakeModel(None), []) == _sha("|-1|-1|mistral3|2x1x4|0:")


def test_fingerprint_changes_with_file_geometry_and_tokens(tmp_path):
    f = tmp_path / "m.gguf"
    f.write_bytes(b"abc")
    m = FakeModel(str(f))
    base = P.fingerprint(m, [1, 2])
    assert P.fingerprint(m, [1, 3]) != base
    m.config.n_kv_heads = 2
    assert P.fingerprint(m, [1, 2]) != base
    m.config.n_kv_heads = 1
    st = os.stat(f)
    os.utime(f, ns=(st.st_atime_ns, st.st_mtime_ns + 100))
    assert P.fingerprint(m, [1, 2]) != base


# ------------------------------------------------------------------ save / load

def _captured(tmp_path, tokens=(3, 1, 4, 1, 5)):
    f = tmp_path / "m.gguf"
    f.write_bytes(b"weights")
    m = FakeModel(str(f))
    return m, jev.SystemPromptCache.capture(m, list(tokens))


def test_capture_leaves_the_prefix_and_round_trips_through_a_file(tmp_path):
    m, c = _captured(tmp_path)
    assert m.cache == [3, 1, 4, 1, 5] and m.ops[:2] == [("reset",), ("prefill", 5)]
    p = tmp_path / "sys.shkv"
    c.save(str(p))
    assert p.read_bytes() == c.to_bytes()
    got = jev.SystemPromptCache.try_load(str(p), m)
    assert got is not None and got.fingerprint == c.fingerprint
    assert np.array_equal(got.tokens, c.tokens) and np.array_equal(got.state, c.state)
    m.reset_kv_cache()
    got.restore_into(m)
    assert m.cache == [3, 1, 4, 1, 5]
    assert got.is_prefix_of([3, 1, 4, 1, 5, 9]) and got.is_prefix_of([3, 1, 4, 1, 5])
    assert not got.is_prefix_of([3, 1, 4, 1]) and not got.is_prefix_of([3, 1, 4, 2, 5, 9])


def test_try_load_misses(tmp_path):
    m, c = _captured(tmp_path)
    good = c.to_bytes()
    hdr = 8 + 1 + 64

    def miss(data):
        p = tmp_path / "x.shkv"
        p.write_bytes(data)
        return jev.SystemPromptCache.try_load(str(p), m) is None

    assert jev.SystemPromptCache.try_load(str(tmp_path / "absent.shkv"), m) is None
    assert miss(b"XXXX" + good[4:])                                        # magic
    assert miss(good[:4] + struct.pack("<i", 2) + good[8:])                 # version
    assert miss(good[:-1])                                                  # truncated payload
    assert miss(good[:hdr + 2])                                             # truncated token list
    assert miss(good[:hdr] + struct.pack("<i", 1_000_001) + good[hdr + 4:])  # token count bound
    assert miss(good[:hdr] + struct.pack("<i", -1) + good[hdr + 4:])
    off = hdr + 4 + 4 * 5
    assert miss(good[:off] + struct.pack("<q", -1) + good[off + 8:])        # state length bound
    assert miss(good[:off] + struct.pack("<q", 2**31) + good[off + 8:])
    other = jev.SystemPromptCache(c.tokens, c.state, P.fingerprint(m, [9, 9]))
    assert miss(other.to_bytes())                                           # another prefix
    assert not miss(good)
    f = tmp_path / "m.gguf"                                                 # the model file changed
    st = os.stat(f)
    os.utime(f, ns=(st.st_atime_ns, st.st_mtime_ns + 10**9))
    assert miss(good)


def test_restore_refuses_another_model(tmp_path):
    m, c = _captured(tmp_path)
    with pytest.raises(jev.InvalidOperationError):
        c.restore_into(FakeModel(str(tmp_path / "other.gguf")))


def test_load_or_capture(tmp_path):
    m, _ = _captured(tmp_path)
    p = str(tmp_path / "sys.shkv")
    first = jev.SystemPromptCache.load_or_capture(m, [2, 7, 1, 8], p)
    assert os.path.exists(p) and ("prefill", 4) in m.ops
    m.ops.clear()
    again = jev.SystemPromptCache.load_or_capture(m, [2, 7, 1, 8], p)
    assert not any(op[0] == "prefill" for op in m.ops)
    assert np.array_equal(again.state, first.state)
    other = jev.SystemPromptCache.load_or_capture(m, [2, 7, 1], p)  # same file, other tokens: recapture
    assert other.token_count == 3 and ("prefill", 3) in m.ops
    ro = tmp_path / "ro"
    ro.mkdir()
    unwritable = str(ro / "missing_dir" / "x.shkv")  # a failed write costs a prefill, not an error
    assert jev.SystemPromptCache.load_or_capture(m, [4, 4], unwritable).token_count == 2


# ------------------------------------------------------------------ decider

SYSTEM = [1, 2, 3, 4, 5]
Q1 = [10, 11, 12, 13]   # instruction and option list of question 1
Q2 = [20, 21, 22]
DOC = [90]              # the "<Document>:" marker after the options
BRANCHES1 = [[60, 61], [62, 63, 64]]
BRANCHES2 = [[70], [71], [72, 73]]
YES, NO = [0, 1], [2]


def _prompt(q, data):
    return SYSTEM + q + DOC + data, SYSTEM + q + DOC


def _decider(size=8):
    m = FakeModel()
    return m, jev.TreeDecider(m, YES, NO, system_tokens=SYSTEM, question_cache_size=size)


def _decide(d, q, data, branches):
    prefix, question = _prompt(q, data)
    return d.decide(prefix, question, branches)


def _cold(q, data, branches):
    return _decide(_decider()[1], q, data, branches)


def test_first_call_restores_the_system_snapshot():
    m, d = _decider()
    assert m.cache == SYSTEM
    r = _decide(d, Q1, [40, 41], BRANCHES1)
    assert r.cached_tokens == len(SYSTEM)  # resident trunk == system: truncate to it
    assert r.prefix_tokens == len(SYSTEM + Q1 + DOC) + 2 and r.suffix_tokens == 5
    assert m.cache == SYSTEM + Q1 + DOC + [40, 41]  # the whole prefix, nothing of the branches
    assert np.isclose(r.probabilities.sum(), 1.0, atol=1e-6)


def test_same_question_new_data_reuses_the_question_prefix():
    m, d = _decider()
    _decide(d, Q1, [40, 41], BRANCHES1)
    warm = _decide(d, Q1, [42, 43, 44], BRANCHES1)
    cold = _cold(Q1, [42, 43, 44], BRANCHES1)
    assert warm.cached_tokens == len(SYSTEM + Q1 + DOC) > cold.cached_tokens == len(SYSTEM)
    assert np.array_equal(warm.margins, cold.margins)
    assert d.question_cache_hits == 0


def test_interleaved_questions_come_back_from_their_snapshots():
    m, d = _decider()
    _decide(d, Q1, [40], BRANCHES1)
    _decide(d, Q2, [50], BRANCHES2)
    restored = _decide(d, Q1, [41, 42], BRANCHES1)
    cold = _cold(Q1, [41, 42], BRANCHES1)
    assert d.question_cache_hits == 1
    assert ("restore", len(SYSTEM + Q1 + DOC)) in m.ops
    assert restored.cached_tokens == len(SYSTEM + Q1 + DOC) > cold.cached_tokens
    assert np.array_equal(restored.margins, cold.margins)


def test_identical_prompt_reruns_its_last_token():
    m, d = _decider()
    a = _decide(d, Q1, [40, 41], BRANCHES1)
    b = _decide(d, Q1, [40, 41], BRANCHES1)
    assert b.cached_tokens == a.prefix_tokens - 1
    assert m.ops[-4:-2] == [("truncate", a.prefix_tokens), ("truncate", a.prefix_tokens - 1)]
    assert np.array_equal(a.margins, b.margins)


def test_snapshot_lru_evicts_the_oldest_and_size_zero_turns_it_off():
    _, d = _decider(size=1)
    _decide(d, Q1, [40], BRANCHES1)
    _decide(d, Q2, [50], BRANCHES2)
    r = _decide(d, Q1, [41], BRANCHES1)   # Q1's snapshot was evicted by Q2's
    assert d.question_cache_hits == 0 and r.cached_tokens == len(SYSTEM)
    m, d = _decider(size=0)
    opened = len(m.ops)  # reset, prefill and snapshot of the system block
    _decide(d, Q1, [40], BRANCHES1)
    _decide(d, Q2, [50], BRANCHES2)
    _decide(d, Q1, [41], BRANCHES1)
    assert d.question_cache_hits == 0 and not any(op[0] == "snapshot" for op in m.ops[opened:])


def test_longest_matching_snapshot_wins_and_moves_to_the_recent_end():
    _, d = _decider(size=2)
    q1b = Q1 + [14, 15]  # a question whose prefix extends Q1's
    _decide(d, Q1, [40], BRANCHES1)
    _decide(d, q1b, [40], BRANCHES1)
    _decide(d, Q2, [50], BRANCHES2)  # evicts Q1's (the oldest)
    r = _decide(d, q1b, [41], BRANCHES1)
    assert d.question_cache_hits == 1 and r.cached_tokens == len(SYSTEM + q1b + DOC)


def test_a_prompt_without_the_system_prefix_starts_cold():
    m, d = _decider()
    r = d.decide([7, 7, 7, 8], [7, 7], BRANCHES1)
    assert r.cached_tokens == 0 and ("reset",) in m.ops[1:]


def test_decider_rejections():
    m = FakeModel()
    with pytest.raises(jev.DataError):
        jev.TreeDecider(m, [], [2])
    d = jev.TreeDecider(m, YES, NO)
    with pytest.raises(jev.ArgumentError):
        d.decide([1, 2], [1], [[3]])


def test_common_prefix_and_temperature_lookup():
    assert jev.common_prefix([1, 2, 3], [1, 2, 4, 5]) == 2
    assert jev.common_prefix([1, 2], [1, 2, 3]) == 2 and jev.common_prefix([], [1]) == 0
    table = {"choice": 2.0, "choice:3-5": 1.5, "noul": 0.0}
    assert jev.temperature_for("choice", 4, table) == 1.5
    assert jev.temperature_for("choice", 2, table) == 2.0
    assert jev.temperature_for("noul", 2, table) == 1e-3
    assert jev.temperature_for("score", 12, table) == 1.0
    assert jev.temperature_for("score", 12) == 1.0
