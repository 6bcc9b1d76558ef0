"""GGUF reader and writer on the host (no GPU).

Mirrors GgufReaderTests.cs: the block geometry table against ggml.h's
constants (the test's own InlineData), a hand-built file whose bytes are
written here independently of jev.gguf's writer, and the rejection of
truncated and non-GGUF files.  The writer is checked by reading its output
back, field by field, and by ModelConfig.FromGguf's key mapping
(ModelConfig.cs:62-112), fallbacks included.
"""
import struct
from dataclasses import fields

import numpy as np
import pytest

import jev
from jev import gguf as G
from helpers import tiny_config

# GgufReaderTests.BlockGeometryMatchesGgml (GgufReaderTests.cs:18-53)
GEOMETRY = [
    ("F32", 1, 4), ("F16", 1, 2), ("BF16", 1, 2), ("Q4_0", 32, 18), ("Q4_1", 32, 20), ("Q5_0", 32, 22),
    ("Q5_1", 32, 24), ("Q8_0", 32, 34), ("Q8_1", 32, 36), ("Q2_K", 256, 84), ("Q3_K", 256, 110),
    ("Q4_K", 256, 144), ("Q5_K", 256, 176), ("Q6_K", 256, 210), ("Q8_K", 256, 292), ("IQ2_XXS", 256, 66),
    ("IQ2_XS", 256, 74), ("IQ2_S", 256, 82), ("IQ3_XXS", 256, 98), ("IQ3_S", 256, 110), ("IQ1_S", 256, 50),
    ("IQ1_M", 256, 56), ("IQ4_NL", 32, 18), ("IQ4_XS", 256, 136), ("TQ1_0", 256, 54), ("TQ2_0", 256, 66),
    ("MXFP4", 32, 17),
]


@pytest.mark.parametrize("name,block,size", GEOMETRY)
def test_block_geometry_matches_ggml(name, block, size):
    tid = G.GGML_TYPES[name][0]
    assert G.block_geometry(tid) == (block, size)


def test_type_ids_are_ggml_h_numbering():
    # the libjev ids used by jev_bind_tensor are the same numbers
    assert G.GGML_TYPES["F32"][0] == jev.TYPE_F32 and G.GGML_TYPES["F16"][0] == jev.TYPE_F16
    assert G.GGML_TYPES["Q4_0"][0] == jev.TYPE_Q4_0 and G.GGML_TYPES["Q5_1"][0] == jev.TYPE_Q5_1
    assert G.GGML_TYPES["Q8_0"][0] == jev.TYPE_Q8_0
    with pytest.raises(G.NotSupportedError):
        G.block_geometry(4)  # a retired id
    with pytest.raises(ValueError):
        G.row_bytes(jev.TYPE_Q8_0, 33)


def _s(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _minimal(weights, version=3, extra_kv=b"", n_extra=0) -> bytes:
    """GgufReaderTests.WriteMinimalGguf (GgufReaderTests.cs:148-184), byte for byte."""
    out = struct.pack("<IIQQ", 0x46554747, version, 1, 6 + n_extra)
    out += _s("general.architecture") + struct.pack("<I", 8) + _s("test")
    out += _s("test.block_count") + struct.pack("<II", 4, 7)
    out += _s("test.scale") + struct.pack("<If", 6, 2.5)
    out += _s("test.flag") + struct.pack("<IB", 7, 1)
    out += _s("test.list") + struct.pack("<IIQ", 9, 8, 3) + _s("a") + _s("b") + _s("c")
    out += _s("test.ints") + struct.pack("<IIQii", 9, 5, 2, 10, 20)
    out += extra_kv
    out += _s("w") + struct.pack("<IQQIQ", 2, 3, 2, 0, 0)
    out += b"\0" * ((32 - len(out) % 32) % 32)
    out += np.asarray(weights, "<f4").tobytes()
    return out


def test_reads_a_hand_built_file(tmp_path):
    p = tmp_path / "tiny.gguf"
    w = [1.0, 2.0, 3.0, 4.0, 5.0, 6.0]
    p.write_bytes(_minimal(w))
    with G.GgufFile(str(p)) as g:
        assert g.version == 3
        assert g.get_string("general.architecture") == "test"
        assert g.get_uint32("test.block_count") == 7
        assert g.get_float32("test.scale") == 2.5
        assert g.get_bool("test.flag") is True
        assert g.get_string_array("test.list") == ["a", "b", "c"]
        assert list(g.metadata["test.ints"]) == [10, 20]
        info = g.get_tensor("w")
        assert info.shape == (3, 2) and info.ggml_type == jev.TYPE_F32
        assert info.element_count == 6 and info.byte_count == 24
        assert info.row_elements == 3 and info.row_count == 2
        assert np.array_equal(g.tensor_bytes(info).view("<f4"), np.asarray(w, np.float32))
        assert g.data_offset % 32 == 0
        with pytest.raises(KeyError):
            g.get_tensor("missing")


def test_rejects_a_truncated_file(tmp_path):
    p = tmp_path / "short.gguf"
    p.write_bytes(_minimal([1.0, 2.0, 3.0, 4.0, 5.0, 6.0])[:-8])  # an interrupted download
    with pytest.raises(OSError, match="incomplete"):
        G.GgufFile(str(p))


def test_rejects_a_non_gguf_file(tmp_path):
    p = tmp_path / "junk.bin"
    p.write_bytes(bytes(range(8)))
    with pytest.raises(jev.DataError):
        G.GgufFile(str(p))
    p.write_bytes(b"")
    with pytest.raises(jev.DataError):
        G.GgufFile(str(p))


def test_rejects_unsupported_and_malformed_headers(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(_minimal([1.0] * 6, version=1))
    with pytest.raises(G.NotSupportedError):
        G.GgufFile(str(p))
    nested = _s("test.nested") + struct.pack("<IIQ", 9, 9, 1)
    p.write_bytes(_minimal([1.0] * 6, extra_kv=nested, n_extra=1))
    with pytest.raises(G.NotSupportedError):
        G.GgufFile(str(p))
    unknown = _s("test.odd") + struct.pack("<I", 13)
    p.write_bytes(_minimal([1.0] * 6, extra_kv=unknown, n_extra=1))
    with pytest.raises(G.NotSupportedError):
        G.GgufFile(str(p))
    huge = struct.pack("<Q", 1 << 40) + b"x"
    p.write_bytes(struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + huge)
    with pytest.raises(jev.DataError, match="implausible"):
        G.GgufFile(str(p))
    p.write_bytes(_minimal([1.0] * 6)[:60])  # header cut inside the metadata
    with pytest.raises(jev.DataError, match="runs past the file"):
        G.GgufFile(str(p))


def test_alignment_key_moves_the_data_section(tmp_path):
    p = tmp_path / "al.gguf"
    data = np.arange(64, dtype=np.float32)
    G.write_gguf(str(p), [("general.architecture", G.STRING, "test")],
                 [G.WriterTensor("v", (64,), jev.TYPE_F32, data)], alignment=256)
    with G.GgufFile(str(p)) as g:
        assert g.get_uint32("general.alignment") == 256
        assert g.data_offset % 256 == 0
        assert np.array_equal(g.tensor_bytes(g.get_tensor("v")).view("<f4"), data)


@pytest.fixture(scope="module")
def synth():
    return jev.SynthModel(tiny_config(), jev.TYPE_Q8_0)


def test_writer_round_trip_of_a_synthetic_checkpoint(tmp_path, synth):
    p = tmp_path / "synth.gguf"
    synth.write_gguf(str(p))
    assert not (tmp_path / "synth.gguf.partial").exists()
    c = synth.config
    with G.GgufFile(str(p)) as g:
        assert len(g.tensors) == 9 * c.n_layers + 2  # tied head: no output.weight
        assert "output.weight" not in g.tensors
        for name, t in synth.tensors.items():
            info = g.get_tensor(name)
            assert info.ggml_type == t.ggml_type
            if t.rows == 1:
                assert info.shape == (t.cols,)
            else:
                assert info.shape == (t.cols, t.rows)  # ne0 = columns, as WeightMatrix.From reads it
            assert (g.data_offset + info.offset) % 32 == 0
            assert np.array_equal(g.tensor_bytes(info), t.data.view(np.uint8))
        assert g.get_uint32("general.file_type") == jev.TYPE_Q8_0
        assert len(g.get_string_array("tokenizer.ggml.tokens")) == c.vocab
        got = G.config_from_gguf(g, initial_kv_capacity=c.initial_kv_capacity)
    for f in fields(c):  # float keys are float32 in the file, as in jev_config
        want = getattr(c, f.name)
        assert getattr(got, f.name) == (np.float32(want) if isinstance(want, float) else want), f.name


def test_config_key_fallbacks_and_yarn(tmp_path):
    p = tmp_path / "cfg.gguf"
    a = "llama."
    md = [("general.architecture", G.STRING, "llama"), (a + "embedding_length", G.UINT32, 256),
          (a + "attention.head_count", G.UINT32, 4), (a + "block_count", G.UINT32, 3),
          (a + "feed_forward_length", G.UINT32, 512), (a + "vocab_size", G.UINT32, 1000),
          (a + "rope.scaling.type", G.STRING, "yarn"), (a + "rope.scaling.factor", G.FLOAT32, 4.0),
          (a + "rope.scaling.original_context_length", G.UINT32, 16384),
          (a + "rope.scaling.beta_fast", G.FLOAT32, 16.0), (a + "rope.scaling.mscale_all_dim", G.FLOAT32, 1.0),
          (a + "rope.scaling.yarn_attn_factor", G.FLOAT32, 0.5), (a + "rope.scaling_beta", G.FLOAT32, 0.1)]
    G.write_gguf(str(p), md, [])
    with G.GgufFile(str(p)) as g:
        c = G.config_from_gguf(g)
    assert (c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim) == (3, 256, 4, 4, 64)
    assert c.vocab == 1000 and c.rope_dim == 64 and c.rope_freq_base == 10000.0 and c.rms_eps == np.float32(1e-5)
    assert c.rope_scaling_yarn == 1 and c.rope_scale_factor == 4.0 and c.rope_original_context == 16384
    assert c.yarn_beta_fast == 16.0 and c.yarn_beta_slow == 1.0 and c.yarn_mscale_all_dim == 1.0
    assert c.rope_attn_factor == 0.5 and c.attention_temperature_scale == np.float32(0.1)

    G.write_gguf(str(p), [("general.architecture", G.STRING, "gpt2")], [])
    with G.GgufFile(str(p)) as g, pytest.raises(G.NotSupportedError):
        G.config_from_gguf(g)
    G.write_gguf(str(p), [], [])
    with G.GgufFile(str(p)) as g, pytest.raises(jev.DataError):
        G.config_from_gguf(g)
    G.write_gguf(str(p), [("general.architecture", G.STRING, "mistral3"),
                          ("mistral3.attention.head_count", G.UINT32, 6),
                          ("mistral3.attention.head_count_kv", G.UINT32, 4)], [])
    with G.GgufFile(str(p)) as g, pytest.raises(jev.DataError, match="do not divide"):
        G.config_from_gguf(g)


def test_writer_rejects_a_short_tensor(tmp_path):
    with pytest.raises(ValueError):
        G.write_gguf(str(tmp_path / "x.gguf"), [], [G.WriterTensor("w", (32, 2), jev.TYPE_Q8_0, np.zeros(67, np.uint8))])
