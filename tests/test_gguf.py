"""The GGUF reader (leat_amd/gguf.py, after leat/gguf.py:64-140) on files whose bytes the tests
place: header, metadata of every value kind, the tensor index with its row-major shapes and
aligned offsets, the data, and the errors leat raises. A Llama GGUF then loads into the decoder
on the GPU and decodes exactly as the model built from the same blocks."""

import struct

import numpy as np
import pytest

from leat_amd.gguf import GGUF, parse
from leat_amd.quant import GGMLType
from tests.gguf_files import f32_bytes, gguf_bytes


def _text(s: str) -> bytes:
    return struct.pack("<Q", len(s)) + s.encode()


def test_parse_hand_built_file(tmp_path):
    # every byte placed here, from the format's layout: version 3, 2 tensors, 4 metadata entries
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 4)
    head += _text("general.architecture") + struct.pack("<I", 8) + _text("llama")
    head += _text("llama.block_count") + struct.pack("<II", 4, 32)
    head += _text("llama.rope.freq_base") + struct.pack("<If", 6, 500000.0)
    head += _text("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 2) + _text("a") + _text("bc")
    # a 2 x 3 F32 tensor at offset 0, a 2 x 64 Q8_0 at 32 (after the 24 bytes, aligned to 32)
    head += _text("norm") + struct.pack("<IQQ", 2, 3, 2) + struct.pack("<IQ", 0, 0)
    head += _text("w") + struct.pack("<IQQ", 2, 64, 2) + struct.pack("<IQ", 8, 32)
    start = -(-len(head) // 32) * 32
    data = bytearray(32 + 4 * 34)
    data[0:24] = np.arange(6, dtype=np.float32).tobytes()
    data[32:] = bytes(range(136))
    path = tmp_path / "hand.gguf"
    path.write_bytes(head + bytes(start - len(head)) + bytes(data))

    g = GGUF.open(path)
    assert g.metadata == {"general.architecture": "llama", "llama.block_count": 32, "llama.rope.freq_base": 500000.0,
                          "tokenizer.ggml.tokens": ["a", "bc"]}  # fmt: skip
    norm, w = g.tensors["norm"], g.tensors["w"]
    assert (norm.type, norm.shape, norm.offset, norm.nbytes) == (GGMLType.F32, (2, 3), start, 24)
    assert (w.type, w.shape, w.offset, w.nbytes) == (GGMLType.Q8_0, (2, 64), start + 32, 136)
    loaded = g.load(device="cpu")
    np.testing.assert_array_equal(loaded["norm"].data.numpy(), np.arange(6, dtype=np.float32))
    assert loaded["w"].data.shape == (4, 34) and bytes(loaded["w"].data.numpy().tobytes()) == bytes(range(136))


def test_alignment_from_metadata(tmp_path):
    blob = gguf_bytes({"general.alignment": 64}, [("a", 0, (3,), f32_bytes([1, 2, 3])), ("b", 0, (2,), f32_bytes([4, 5]))],
                      alignment=64)  # fmt: skip
    path = tmp_path / "a.gguf"
    path.write_bytes(blob)
    g = GGUF.open(path)
    assert g.tensors["a"].offset % 64 == 0 and g.tensors["b"].offset - g.tensors["a"].offset == 64
    np.testing.assert_array_equal(g.load("cpu")["b"].data.numpy(), [4.0, 5.0])


def test_version_2_and_errors(tmp_path):
    ok = gguf_bytes({"x": 1}, [("t", 0, (4,), f32_bytes([0, 1, 2, 3]))], version=2)
    assert parse(memoryview(ok))[1]["t"].shape == (4,)
    with pytest.raises(ValueError, match="not a GGUF"):
        parse(memoryview(b"GGML" + ok[4:]))
    with pytest.raises(ValueError, match="version 1"):
        parse(memoryview(ok[:4] + struct.pack("<I", 1) + ok[8:]))
    with pytest.raises(ValueError, match="unknown ggml type"):
        parse(memoryview(gguf_bytes({}, [("t", 77, (4,), bytes(16))])))
    with pytest.raises(ValueError, match="not whole blocks"):  # Q4_K rows of 100 weights
        parse(memoryview(gguf_bytes({}, [("t", 12, (1, 100), bytes(144))])))
    with pytest.raises(ValueError, match="power of 2"):
        parse(memoryview(gguf_bytes({"general.alignment": 48}, [("t", 0, (4,), bytes(16))])))
    with pytest.raises(ValueError, match="unknown metadata value type"):
        parse(memoryview(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + _text("k") + struct.pack("<I", 13)))
    path = tmp_path / "short.gguf"
    path.write_bytes(gguf_bytes({}, [("t", 0, (64,), bytes(256))])[:-8])
    with pytest.raises(ValueError, match="truncated"):
        GGUF.open(path)


@pytest.mark.gpu
def test_llama_gguf_decodes_as_built(cuda, tmp_path):
    # a small Llama's blocks written into a GGUF with llama.* metadata and rope_freqs: the decoder
    # loaded from it gives the same logits, bit for bit, as the one built from the blocks
    import torch

    from leat_amd.model import LlamaConfig, Model, from_gguf, llama3_rope_factors, synthetic

    cfg = LlamaConfig(dim=512, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=1024, vocab=1000, context=128,
                      rope_theta=500000.0, rope_scaling=(8.0, 1.0, 4.0, 32))  # fmt: skip
    w = synthetic(cfg, seed=9)
    built = Model(cfg, w)

    def raw(q):
        return q.data.cpu().numpy().tobytes()

    tensors = [("token_embd.weight", 12, (cfg.vocab, cfg.dim), raw(w.embed)),
               ("output_norm.weight", 0, (cfg.dim,), raw(w.output_norm)), ("output.weight", 14, (cfg.vocab, cfg.dim), raw(w.output)),
               ("rope_freqs.weight", 0, (64,), f32_bytes(llama3_rope_factors(128, cfg.rope_theta, cfg.rope_scaling)))]  # fmt: skip
    for i, l in enumerate(w.layers):
        tensors += [(f"blk.{i}.attn_norm.weight", 0, (cfg.dim,), raw(l.attn_norm)),
                    (f"blk.{i}.attn_q.weight", 12, l.q.shape, raw(l.q)), (f"blk.{i}.attn_k.weight", 12, l.k.shape, raw(l.k)),
                    (f"blk.{i}.attn_v.weight", 12, l.v.shape, raw(l.v)), (f"blk.{i}.attn_output.weight", 12, l.o.shape, raw(l.o)),
                    (f"blk.{i}.ffn_norm.weight", 0, (cfg.dim,), raw(l.ffn_norm)),
                    (f"blk.{i}.ffn_gate.weight", 12, l.gate.shape, raw(l.gate)), (f"blk.{i}.ffn_up.weight", 12, l.up.shape, raw(l.up)),
                    (f"blk.{i}.ffn_down.weight", 14, l.down.shape, raw(l.down))]  # fmt: skip
    meta = {"general.architecture": "llama", "llama.embedding_length": cfg.dim, "llama.block_count": cfg.layers,
            "llama.attention.head_count": cfg.heads, "llama.attention.head_count_kv": cfg.kv_heads,
            "llama.feed_forward_length": cfg.ffn, "llama.rope.freq_base": cfg.rope_theta,
            "llama.attention.layer_norm_rms_epsilon": cfg.norm_eps}  # fmt: skip
    path = tmp_path / "tiny.gguf"
    path.write_bytes(gguf_bytes(meta, tensors))
    loaded = from_gguf(path, context=cfg.context)
    assert loaded.config.vocab == cfg.vocab and loaded.config.kv_heads == 2
    slots = torch.zeros(1, dtype=torch.int32, device=cuda)
    for pos, token in enumerate([3, 999, 17]):
        ids = torch.tensor([token], dtype=torch.int32, device=cuda)
        at = torch.tensor([pos], dtype=torch.int32, device=cuda)
        np.testing.assert_array_equal(loaded.logits(ids, slots, at).cpu().numpy(), built.logits(ids, slots, at).cpu().numpy())
