"""SystemPromptCache (src/Jevstral/SystemPromptCache.cs) over the device KV cache.

A snapshot of the keys and values a prefill of a fixed token prefix leaves in
the cache.  Attention is causal, so those positions depend on nothing after
them: restoring the snapshot and running the rest of a prompt gives the same
bits as running the whole prompt (the kernels are batch-invariant).  The
snapshot is tied by a fingerprint to the model file, the cache geometry and
the tokens, and is persisted in the reference's SHKV format
(SystemPromptCache.cs:114-131), so a file written by either runtime loads in
the other.

SHKV version 1, little-endian, as .NET's BinaryWriter writes it:
  uint32 magic 0x53484B56 ("SHKV"), int32 version 1,
  string fingerprint (7-bit encoded byte length, then UTF-8),
  int32 token count, int32 tokens[count],
  int64 state length, float32 state[length]   (KvCache.Snapshot's flat layout)
"""
from __future__ import annotations

import hashlib
import os
import struct
from typing import Optional, Sequence

import numpy as np

MAGIC = 0x53484B56  # "SHKV" (SystemPromptCache.cs:25)
FORMAT_VERSION = 1  # SystemPromptCache.cs:26
_UNIX_EPOCH_TICKS = 621_355_968_000_000_000  # DateTime(1970, 1, 1).Ticks: 100 ns units since 0001-01-01
_MAX_TOKENS = 1_000_000  # TryLoad's bound (SystemPromptCache.cs:148)
_INT32_MAX = 2**31 - 1


class InvalidOperationError(RuntimeError):
    """InvalidOperationException: a snapshot restored into the wrong model or prefix."""


def encode_dotnet_string(s: str) -> bytes:
    """BinaryWriter.Write(string): the UTF-8 byte count as a 7-bit encoded
    integer (low 7 bits first, high bit = more follows), then the bytes."""
    b = s.encode("utf-8")
    n, out = len(b), bytearray()
    while n >= 0x80:
        out.append((n & 0x7F) | 0x80)
        n >>= 7
    out.append(n)
    return bytes(out) + b


def _read_exact(f, n: int) -> bytes:
    b = f.read(n)
    if len(b) != n:
        raise EOFError("end of stream")  # EndOfStreamException
    return b


def _read_dotnet_string(f) -> str:
    """BinaryReader.ReadString: at most five length bytes (a 32-bit count)."""
    n, shift = 0, 0
    while True:
        byte = _read_exact(f, 1)[0]
        n |= (byte & 0x7F) << shift
        if byte < 0x80:
            break
        shift += 7
        if shift >= 35:
            raise ValueError("bad 7-bit encoded string length")  # FormatException: not a miss
    if n > _INT32_MAX:
        raise ValueError("bad 7-bit encoded string length")
    return _read_exact(f, n).decode("utf-8", errors="replace")


def _file_identity(path: Optional[str]):
    """FileInfo(ModelPath): Name, Length and LastWriteTimeUtc.Ticks, or -1
    for a file that does not exist (SystemPromptCache.cs:92-98)."""
    if not path:
        return "", -1, -1
    name = os.path.basename(path)
    try:
        st = os.stat(path)
    except OSError:
        return name, -1, -1
    if not os.path.isfile(path):
        return name, -1, -1
    ticks = _UNIX_EPOCH_TICKS + st.st_mtime_ns // 100
    return name, st.st_size, ticks


def fingerprint(model, tokens: Sequence[int]) -> str:
    """ComputeFingerprint (SystemPromptCache.cs:90-104): SHA-256, lower-case
    hex, of "name|length|ticks|arch|LxKVxHD|count:t0,t1,...," in UTF-8."""
    name, length, ticks = _file_identity(getattr(model, "model_path", None))
    c = model.config
    toks = np.asarray(tokens, dtype=np.int64).ravel()
    text = (f"{name}|{length}|{ticks}|{c.architecture}|{c.n_layers}x{c.n_kv_heads}x{c.head_dim}|"
            f"{len(toks)}:" + "".join(f"{int(t)}," for t in toks))
    return hashlib.sha256(text.encode("utf-8")).hexdigest()


class SystemPromptCache:
    """A captured prefix: its tokens, the flat KV state and the fingerprint."""

    def __init__(self, tokens: Sequence[int], state: np.ndarray, fingerprint_hex: str, device=None):
        self.tokens = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).ravel())
        self.state = np.ascontiguousarray(np.asarray(state, dtype=np.float32).ravel())
        self.fingerprint = fingerprint_hex
        # the same state kept in HBM (a DeviceSnapshot of the model it was
        # captured or first restored into): later restores copy inside device memory
        self._device = device
        self._device_model = None

    @property
    def token_count(self) -> int:
        return int(self.tokens.size)

    @property
    def byte_size(self) -> int:
        return int(self.state.size) * 4

    @classmethod
    def capture(cls, model, tokens: Sequence[int]) -> "SystemPromptCache":
        """CaptureAsync (SystemPromptCache.cs:51-60): prefill into a reset
        cache; the model's cache is left holding exactly the prefix."""
        toks = np.asarray(tokens, dtype=np.int32).ravel()
        model.reset_kv_cache()
        model.prefill(toks)
        take_device = getattr(model, "kv_snapshot_device", None)
        device = take_device(len(toks)) if take_device else None
        host = device.to_host() if device is not None else model.kv_snapshot(len(toks))
        cache = cls(toks, host, fingerprint(model, toks), device)
        cache._device_model = model if device is not None else None
        return cache

    def restore_into(self, model) -> None:
        """RestoreInto (SystemPromptCache.cs:67-75): refuses a snapshot taken
        under a different model file, geometry or prefix."""
        expected = fingerprint(model, self.tokens)
        if expected != self.fingerprint:
            raise InvalidOperationError(
                f"This snapshot was captured for a different model or prefix "
                f"(fingerprint {self.fingerprint}, model reports {expected}).")
        if self._device is not None and self._device_model is model:
            model.kv_restore(self._device)
            return
        model.kv_restore(self.state, self.token_count)
        take_device = getattr(model, "kv_snapshot_device", None)
        if take_device is not None:
            if self._device is not None:
                self._device.close()
            self._device, self._device_model = take_device(self.token_count), model

    def is_prefix_of(self, tokens: Sequence[int]) -> bool:
        """IsPrefixOf (SystemPromptCache.cs:81-82)."""
        t = np.asarray(tokens, dtype=np.int64).ravel()
        n = self.token_count
        return t.size >= n and bool(np.array_equal(t[:n], self.tokens.astype(np.int64)))

    # ------------------------------------------------------------ persistence
    def _header(self) -> bytes:
        return (struct.pack("<Ii", MAGIC, FORMAT_VERSION) + encode_dotnet_string(self.fingerprint)
                + struct.pack("<i", self.token_count) + self.tokens.astype("<i4").tobytes()
                + struct.pack("<q", int(self.state.size)))

    def to_bytes(self) -> bytes:
        """The SHKV file's bytes."""
        return self._header() + self.state.astype("<f4").tobytes()

    def save(self, path: str) -> None:
        """Save (SystemPromptCache.cs:114-131): header, then one bulk write of the floats."""
        with open(path, "wb") as f:
            f.write(self._header())
            f.write(self.state.astype("<f4").tobytes())

    @classmethod
    def try_load(cls, path: str, model) -> Optional["SystemPromptCache"]:
        """TryLoad (SystemPromptCache.cs:138-169): None when the file is absent,
        unreadable, truncated, of another format or version, or captured under
        a different model or prefix -- a stale cache is a miss, not an error."""
        try:
            with open(path, "rb") as f:
                magic, version = struct.unpack("<Ii", _read_exact(f, 8))
                if magic != MAGIC or version != FORMAT_VERSION:
                    return None
                fp = _read_dotnet_string(f)
                (count,) = struct.unpack("<i", _read_exact(f, 4))
                if count < 0 or count > _MAX_TOKENS:
                    return None
                tokens = np.frombuffer(_read_exact(f, 4 * count), dtype="<i4").astype(np.int32)
                (length,) = struct.unpack("<q", _read_exact(f, 8))
                if length < 0 or length > _INT32_MAX:
                    return None
                state = np.frombuffer(_read_exact(f, 4 * length), dtype="<f4").astype(np.float32)
        except (OSError, EOFError):  # IOException, EndOfStreamException, UnauthorizedAccessException
            return None
        cache = cls(tokens, state, fp)
        if fingerprint(model, tokens) != fp:
            return None
        return cache

    @classmethod
    def load_or_capture(cls, model, tokens: Sequence[int], path: str) -> "SystemPromptCache":
        """LoadOrCaptureAsync (SystemPromptCache.cs:176-191): the file's
        snapshot when it is valid for exactly these tokens, else a fresh
        capture written back (a write failure costs a prefill, not an error)."""
        toks = np.asarray(tokens, dtype=np.int32).ravel()
        cached = cls.try_load(path, model)
        if cached is not None and np.array_equal(cached.tokens, toks):
            return cached
        fresh = cls.capture(model, toks)
        try:
            fresh.save(path)
        except OSError:
            pass
        return fresh
