"""The decode step around the quantized products on a gfx950 GPU against the CPU oracle: the
embedding gather, RoPE with the KV store, FlashDecoding attention, argmax, and whole decode steps
of a small Llama-architecture model (eager and as a replayed HIP graph).

Shapes, seeds and tolerances follow leat's kernel tests (tests/test_kernels.py:470-560, 692-730,
928-933); the model's step is compared at leat's model-level tolerance, 2e-3
(tests/test_model.py:46-52).
"""

import numpy as np
import pytest
import torch

from leat_amd import kernels, ops
from leat_amd.model import GraphStep, LlamaConfig, Model, llama3_rope_factors, rope_table, synthetic
from leat_amd.quant import GGMLType
from oracle import leat_oracle as O
from tests.conftest import assert_close, gpu, host, make_weights, normal

pytestmark = pytest.mark.gpu
SLOTS = 3


@pytest.mark.parametrize("ggml_type", [GGMLType.Q4_K, GGMLType.Q6_K, GGMLType.Q8_0])
def test_embedding(cuda, ggml_type):
    # rows of the token ids decoded bit for bit as the dequantizer decodes them; ids outside the
    # matrix give zeros
    rng = np.random.default_rng(60)
    vocab, dim = 300, 512
    w = make_weights(ggml_type, vocab, dim, rng)
    ids = np.array([0, 299, 17, 17, 150], np.int32)
    got = host(kernels.embedding(gpu(ids), w.q))
    want = O.dequant(int(ggml_type), w.blocks, vocab, dim)[ids]
    np.testing.assert_array_equal(got, want)
    assert (host(kernels.embedding(gpu(np.array([-1, 300], np.int32)), w.q)) == 0).all()


@pytest.mark.parametrize("halves", [False, True])
@pytest.mark.parametrize("rotated", [128, 64])
def test_rotate(cuda, halves, rotated):
    # leat's test_rotate_rows shape (tests/test_kernels.py:734-760): tokens at positions of slots of
    # their own or sharing one; q rotated in f32 against the f64 rotation, the cache's f16 keys and
    # values within one f16 step of the oracle's
    rng = np.random.default_rng(19)
    rows, dim, heads, kv_heads = [(0, 7), (2, 300), (1, 511), (2, 3)], 128, 32, 8
    q, k, v = (normal(rng, 1, len(rows), h, dim) for h in (heads, kv_heads, kv_heads))
    angles = rng.uniform(0, 6, (512, rotated // 2)).astype(np.float32)
    cos, sin = np.cos(angles), np.sin(angles)
    cache = torch.zeros(2, SLOTS, kv_heads, 512, dim, dtype=torch.float16, device=cuda)
    spans = [ops.Span(s, p) for s, p in rows]
    out, cache = ops.rotate(gpu(q), gpu(k), gpu(v), cache, spans, ((gpu(cos), gpu(sin)), rotated), halves)
    out, stored = host(out)[0], host(cache)
    for t, (slot, pos) in enumerate(rows):
        want_q = O.rotary(q[0, t], cos[pos], sin[pos], halves)
        np.testing.assert_allclose(out[:, t], want_q, rtol=1e-6, atol=1e-6)
        want_k = O.rotary(k[0, t], cos[pos], sin[pos], halves).astype(np.float16)
        got_k = stored[0, slot, :, pos]
        steps = np.abs(got_k.view(np.int16).astype(np.int32) - want_k.view(np.int16).astype(np.int32))
        assert steps.max() <= 1 and np.count_nonzero(steps) <= 4
        np.testing.assert_array_equal(stored[1, slot, :, pos], v[0, t].astype(np.float16))
    # the reference semantics store the same cache, and rotate q within f32 rounding
    ref_cache = torch.zeros_like(cache)
    import os

    os.environ["LEAT_KERNELS"] = "ref"
    try:
        ref_out, ref_cache = ops.rotate(gpu(q), gpu(k), gpu(v), ref_cache, spans, ((gpu(cos), gpu(sin)), rotated), halves)
    finally:
        del os.environ["LEAT_KERNELS"]
    np.testing.assert_allclose(host(ref_out)[0], out, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(host(ref_cache).astype(np.float32), stored.astype(np.float32), rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("rotated", [128, 64])
@pytest.mark.parametrize("rows", [[(1, 37)], [(0, 5), (2, 511)], [(1, 600)]])
def test_qkv_rotate_fused(cuda, rows, rotated):
    # the q, k, v products with RoPE and the KV store in one launch (leat_qkv_rotate_f32) against
    # linears() then rotate(): q and the whole cache bit for bit, at Llama-3-8B's attention shapes
    # (32 heads, 8 kv heads of 128, 4096 columns of Q4_K); a position past the cache (600 of 512)
    # stores nothing in either
    rng = np.random.default_rng(len(rows) + rotated)
    heads, kv_heads, dim, cols, positions = 32, 8, 128, 4096, 512
    wq, wk, wv = (make_weights(GGMLType.Q4_K, n * dim, cols, rng, synthetic=True).q for n in (heads, kv_heads, kv_heads))
    x = gpu(normal(rng, 1, len(rows), cols, scale=2.0))
    norm = (gpu(rng.uniform(0.5, 1.5, cols).astype(np.float32)), 1e-5)
    angles = rng.uniform(0, 6, (positions, rotated // 2)).astype(np.float32)
    rope = ((gpu(np.cos(angles)), gpu(np.sin(angles))), rotated)
    spans = [ops.Span(s, p) for s, p in rows]
    fused = torch.zeros(2, SLOTS, kv_heads, positions, dim, dtype=torch.float16, device=cuda)
    split = torch.zeros_like(fused)
    assert kernels.supports_qkv_rotate(x, wq, wk, wv, fused, False, norm)
    got = host(ops.qkv_rotate(x, wq, wk, wv, norm, fused, spans, rope, False))
    q, k, v = ops.linears(x, wq, wk, wv, norm=norm)
    T = len(rows)
    want, _ = ops.rotate(q.reshape(1, T, heads, dim), k.reshape(1, T, kv_heads, dim), v.reshape(1, T, kv_heads, dim),
                         split, spans, rope, False)  # fmt: skip
    want = host(want)
    for t, (_, pos) in enumerate(rows):
        if pos < positions:
            np.testing.assert_array_equal(got[:, :, t], want[:, :, t])
    np.testing.assert_array_equal(host(fused).view(np.uint16), host(split).view(np.uint16))
    assert host(fused).any() == any(pos < positions for _, pos in rows)


# cache positions and lengths of leat's test_attention (tests/test_kernels.py:493-511)
@pytest.mark.parametrize("n, length", [(64, 1), (64, 64), (1024, 63), (1024, 65), (1024, 1000), (3072, 3072),
                                       (4096, 3079), (4096, 4096), (16384, 9000)])  # fmt: skip
def test_attention(cuda, n, length):
    rng = np.random.default_rng(length)
    cache = rng.standard_normal((2, SLOTS, 8, n, 128)).astype(np.float16)
    q = normal(rng, 1, 32, 1, 128)
    got = host(ops.attention(gpu(q), gpu(cache), [ops.Span(1, length - 1)], 128**-0.5))[0, 0].reshape(32, 128)
    want = O.attention(q[0, :, 0], cache[0, 1, :, :length], cache[1, 1, :, :length], 128**-0.5)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=2e-3)
    assert_close(got, want, 1e-4)


@pytest.mark.parametrize("heads, kv_heads", [(16, 2), (8, 8), (32, 16)])
def test_attention_rows(cuda, heads, kv_heads):
    # a decode step's rows, each its own slot and length (two in one slot); GQA groups of 8, 1, 2
    rng = np.random.default_rng(heads)
    rows = [(0, 7), (2, 300), (1, 4095), (2, 1)]
    cache = rng.standard_normal((2, SLOTS, kv_heads, 4096, 128)).astype(np.float16)
    q = normal(rng, 1, heads, len(rows), 128, scale=0.3)
    spans = [ops.Span(s, p) for s, p in rows]
    assert kernels.supports_attention(gpu(q), gpu(cache))
    got = host(ops.attention(gpu(q), gpu(cache), spans, 0.1))[0].reshape(len(rows), heads, 128)
    for t, (slot, pos) in enumerate(rows):
        want = O.attention(q[0, :, t], cache[0, slot, :, : pos + 1], cache[1, slot, :, : pos + 1], 0.1)
        np.testing.assert_allclose(got[t], want, rtol=2e-3, atol=2e-3)
        assert_close(got[t], want, 1e-4)


@pytest.mark.parametrize("max_length", [128, 129, 2048, 2049])
@pytest.mark.parametrize("heads, kv_heads", [(8, 8), (8, 4), (16, 4), (16, 2)])
def test_attention_wave_keys(cuda, heads, kv_heads, max_length):
    # launches of 129 .. 2048 keys take 8 keys a wave (64-key chunks), the others 16 (128-key
    # chunks): rows ending either side of both chunk sizes, in every query-group size
    rng = np.random.default_rng(max_length + heads + kv_heads)
    cache = rng.standard_normal((2, SLOTS, kv_heads, 2560, 128)).astype(np.float16)
    rows = [(s, p) for s, p in [(0, 0), (1, 63), (2, 64), (0, 127), (1, 128), (2, 1000), (0, 2047), (1, 2048)]
            if p < max_length]  # fmt: skip
    q = normal(rng, 1, heads, len(rows), 128, scale=0.3)
    slots, lengths = [s for s, _ in rows], [p + 1 for _, p in rows]
    got = host(kernels.attention(gpu(q), gpu(cache), slots, lengths, 0.1, max_length))[0]
    got = got.reshape(len(rows), heads, 128)
    for t, (slot, pos) in enumerate(rows):
        want = O.attention(q[0, :, t], cache[0, slot, :, : pos + 1], cache[1, slot, :, : pos + 1], 0.1)
        np.testing.assert_allclose(got[t], want, rtol=2e-3, atol=2e-3)
        assert_close(got[t], want, 1e-4)


def test_attention_workspace_reuse(cuda):
    # one workspace serves calls of as many rows or fewer one after another
    rng = np.random.default_rng(5)
    heads, kv_heads, n = 16, 4, 2048
    cache = rng.standard_normal((2, SLOTS, kv_heads, n, 128)).astype(np.float16)
    device_cache = gpu(cache)
    work = kernels.attention_workspace(4, heads, n, cuda)
    for rows in ([(0, 2047), (1, 5), (2, 300), (0, 1000)], [(2, 129)], [(1, 0), (0, 700), (2, 2047)],
                 [(0, 2047), (1, 127), (2, 128), (1, 1500)]):  # fmt: skip
        q = normal(rng, 1, heads, len(rows), 128, scale=0.3)
        slots, lengths = [s for s, _ in rows], [p + 1 for _, p in rows]
        got = host(kernels.attention(gpu(q), device_cache, slots, lengths, 0.1, n, work))[0]
        got = got.reshape(len(rows), heads, 128)
        for t, (slot, pos) in enumerate(rows):
            want = O.attention(q[0, :, t], cache[0, slot, :, : pos + 1], cache[1, slot, :, : pos + 1], 0.1)
            np.testing.assert_allclose(got[t], want, rtol=2e-3, atol=2e-3)


def test_attention_workspace_for_longer_rows(cuda):
    # a workspace sized for rows of up to 3000 keys (128-key chunks) serves launches of 2048, 1000
    # and 129 keys, which take more, shorter chunks
    rng = np.random.default_rng(9)
    heads, kv_heads, n = 16, 4, 3000
    cache = rng.standard_normal((2, SLOTS, kv_heads, n, 128)).astype(np.float16)
    device_cache = gpu(cache)
    work = kernels.attention_workspace(2, heads, n, cuda)
    for max_length, rows in ((2048, [(0, 2047), (1, 700)]), (1000, [(2, 999)]), (129, [(1, 128), (0, 3)]),
                             (3000, [(0, 2999), (2, 64)])):  # fmt: skip
        q = normal(rng, 1, heads, len(rows), 128, scale=0.3)
        slots, lengths = [s for s, _ in rows], [p + 1 for _, p in rows]
        got = host(kernels.attention(gpu(q), device_cache, slots, lengths, 0.1, max_length, work))[0]
        got = got.reshape(len(rows), heads, 128)
        for t, (slot, pos) in enumerate(rows):
            want = O.attention(q[0, :, t], cache[0, slot, :, : pos + 1], cache[1, slot, :, : pos + 1], 0.1)
            np.testing.assert_allclose(got[t], want, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("heads, kv_heads", [(32, 8), (16, 16), (16, 2)])
def test_attention_q8_is_quantize_q8(cuda, heads, kv_heads):
    # leat_attention_q8: the f32 output bit for bit leat_attention's, and its q8 bit for bit
    # quantize_q8 of that output, on rows of one chunk (written by the partial kernel) and of many
    # (by the combine), a row with no keys, and a slot outside the cache
    rng = np.random.default_rng(heads + kv_heads)
    n = 2048
    cache = gpu(rng.standard_normal((2, SLOTS, kv_heads, n, 128)).astype(np.float16))
    rows = [(0, 0), (1, 127), (2, 128), (0, 2047), (1, 600), (2, -1), (9, 10)]  # (slot, length)
    q = gpu(normal(rng, 1, heads, len(rows), 128, scale=0.3))
    slots, lengths = [s for s, _ in rows], [max(p, 0) for _, p in rows]
    want = kernels.attention(q, cache, slots, lengths, 0.1, n)
    got, (hq, hd, hs) = kernels.attention_q8(q, cache, slots, lengths, 0.1, n)
    np.testing.assert_array_equal(host(got), host(want))
    wq, wd, ws = kernels.quantize_q8(want.reshape(len(rows), heads * 128))
    np.testing.assert_array_equal(host(hq), host(wq))
    np.testing.assert_array_equal(host(hd), host(wd))
    np.testing.assert_array_equal(host(hs), host(ws))


@pytest.mark.parametrize("tokens", [1, 2, 3, 8])
def test_attention_linear_is_attention_then_linear(cuda, tokens):
    # ops.attention_linear: the o product from the attention kernels' own q8, bit for bit the
    # product of the attention output through ops.linear (which quantizes it again), residual in
    rng = np.random.default_rng(70 + tokens)
    heads, kv_heads, n = 32, 8, 1024
    cache = gpu(rng.standard_normal((2, SLOTS, kv_heads, n, 128)).astype(np.float16))
    wo = make_weights(GGMLType.Q4_K, 512, heads * 128, rng, synthetic=True)
    q = gpu(normal(rng, 1, heads, tokens, 128, scale=0.3))
    residual = gpu(normal(rng, 1, tokens, 512))
    slots = torch.tensor([t % SLOTS for t in range(tokens)], dtype=torch.int32, device=cuda)
    lengths = torch.tensor([1 + 131 * t for t in range(tokens)], dtype=torch.int32, device=cuda)
    got = ops.attention_linear(q, cache, None, 0.1, wo.q, residual, slots, lengths, n)
    att = ops.attention(q, cache, None, 0.1, slots, lengths, n)
    np.testing.assert_array_equal(host(got), host(ops.linear(att, wo.q, residual=residual)))


@pytest.mark.parametrize("rows, n", [(1, 128256), (5, 32000), (2, 300)])
def test_argmax(cuda, rows, n):
    # leat's test_argmax (tests/test_kernels.py:926-933): many ties, the first must win; -inf
    # columns; and NaN, never chosen
    rng = np.random.default_rng(n)
    x = rng.integers(-50, 50, (rows, n)).astype(np.float32)
    x[:, ::7] = -np.inf
    x[:, 5::11] = np.nan
    got = host(ops.argmax(gpu(x)))[:, 0]
    np.testing.assert_array_equal(got, O.argmax(x))


# ---------------------------------------------------------------- whole decode steps

TINY = LlamaConfig(dim=512, layers=2, heads=8, kv_heads=2, head_dim=128, ffn=1024, vocab=1000, context=256,
                   rope_theta=10000.0, rope_scaling=(8.0, 1.0, 4.0, 64))  # fmt: skip


def _oracle_model(weights, config):
    def blocks(q):
        return host(q.data).reshape(-1, q.data.shape[-1])

    layers = [{"attn_norm": host(l.attn_norm), "q": blocks(l.q), "k": blocks(l.k), "v": blocks(l.v), "o": blocks(l.o),
               "ffn_norm": host(l.ffn_norm), "gate": blocks(l.gate), "up": blocks(l.up), "down": blocks(l.down)}
              for l in weights.layers]  # fmt: skip
    factors = llama3_rope_factors(config.head_dim, config.rope_theta, config.rope_scaling)
    types = {"embed": O.Q4_K, "output": O.Q6_K, "q": O.Q4_K, "k": O.Q4_K, "v": O.Q4_K, "o": O.Q4_K, "gate": O.Q4_K,
             "up": O.Q4_K, "down": O.Q6_K}  # fmt: skip
    return {"embed": blocks(weights.embed), "output": blocks(weights.output), "output_norm": host(weights.output_norm),
            "layers": layers, "types": types,
            "rope": O.rope_table(config.head_dim, config.rope_theta, config.context, factors)}  # fmt: skip


def test_rope_tables_match_oracle(cuda):
    factors = llama3_rope_factors(128, 500000.0, (8.0, 1.0, 4.0, 8192))
    assert factors[0] == 1.0 and factors[-1] == 8.0 and all(a <= b for a, b in zip(factors, factors[1:]))
    cos, sin = rope_table(128, 500000.0, 4096, factors, "cuda")
    want_cos, want_sin = O.rope_table(128, 500000.0, 4096, factors)
    np.testing.assert_array_equal(host(cos), want_cos)
    np.testing.assert_array_equal(host(sin), want_sin)


def test_decode_steps_against_oracle(cuda):
    # a prompt's tokens fed one decode step at a time into slot 0, then greedy steps: each step's
    # logits within 2e-3 of the oracle's (which keeps its own f16 cache), and the greedy token the
    # oracle's wherever its top two logits are apart by more than that
    weights = synthetic(TINY, seed=3)
    model = Model(TINY, weights)
    oracle = _oracle_model(weights, TINY)
    cache = np.zeros((TINY.layers, 2, TINY.kv_heads, TINY.context, TINY.head_dim), np.float16)
    slots = torch.zeros(1, dtype=torch.int32, device=cuda)
    token = 17
    for pos in range(12):
        logits = host(model.logits(torch.tensor([token], dtype=torch.int32, device=cuda), slots,
                                   torch.tensor([pos], dtype=torch.int32, device=cuda)))[0]  # fmt: skip
        want = O.decode_logits(oracle, cache, token, pos, {"dim": TINY.dim, "heads": TINY.heads,
                               "kv_heads": TINY.kv_heads, "head_dim": TINY.head_dim, "eps": TINY.norm_eps,
                               "vocab": TINY.vocab})  # fmt: skip
        assert_close(logits, want, 2e-3)
        top2 = np.sort(want)[-2:]
        if top2[1] - top2[0] > 4e-3 * np.abs(want).max():
            assert int(np.argmax(logits)) == int(np.argmax(want))
        token = int(np.argmax(want)) if pos >= 6 else (31 * pos + 5) % TINY.vocab


def test_graph_step_replays_eager(cuda):
    # two rows (slots 0 and 1) decoded by a captured step that advances itself, against the same
    # steps run eagerly on a copy of the cache: the same tokens, replay after replay
    weights = synthetic(TINY, seed=4)
    cfg = LlamaConfig(**{**TINY.__dict__, "slots": 2})
    graphed, eager = Model(cfg, weights), Model(cfg, weights)
    step = GraphStep(graphed, 2)
    step.tokens.copy_(torch.tensor([5, 9], dtype=torch.int32))
    step.slots.copy_(torch.arange(2, dtype=torch.int32))
    step.positions.zero_()
    tokens = torch.tensor([5, 9], dtype=torch.int32, device=cuda)
    slots = torch.arange(2, dtype=torch.int32, device=cuda)
    for pos in range(6):
        step.replay()
        nxt = eager.step(tokens, slots, torch.full((2,), pos, dtype=torch.int32, device=cuda))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(step.next), host(nxt))
        np.testing.assert_array_equal(host(step.tokens), host(nxt))
        assert host(step.positions).tolist() == [pos + 1, pos + 1]
        tokens = nxt.clone()
    for a, b in zip(graphed.cache, eager.cache, strict=True):
        np.testing.assert_array_equal(host(a)[:, :, :, :6], host(b)[:, :, :, :6])


def test_graph_step_length_buckets(cuda):
    # replays that name their rows' longest length run the short-context graph (one attention
    # chunk, no combine) up to 128 keys and the context's past it: positions 120..135 cross the
    # boundary, every step the eager step's tokens bit for bit
    weights = synthetic(TINY, seed=6)
    cfg = LlamaConfig(**{**TINY.__dict__, "slots": 2})
    graphed, eager = Model(cfg, weights), Model(cfg, weights)
    step = GraphStep(graphed, 2)
    assert step.buckets == (128, TINY.context)
    rng = np.random.default_rng(8)
    start = 120
    prompt = rng.integers(0, TINY.vocab, (2, start)).astype(np.int32)
    for model in (graphed, eager):  # the same cache up to position 119 in both
        for row in range(2):
            ids = torch.tensor(prompt[row], dtype=torch.int32, device=cuda)
            model.step(ids, torch.full((start,), row, dtype=torch.int32, device=cuda),
                       torch.arange(start, dtype=torch.int32, device=cuda), last=True)  # fmt: skip
    tokens = torch.tensor([5, 9], dtype=torch.int32, device=cuda)
    step.tokens.copy_(tokens)
    step.slots.copy_(torch.arange(2, dtype=torch.int32))
    step.positions.fill_(start)
    slots = torch.arange(2, dtype=torch.int32, device=cuda)
    for pos in range(start, start + 16):
        step.replay(max_length=pos + 1)
        nxt = eager.step(tokens, slots, torch.full((2,), pos, dtype=torch.int32, device=cuda))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(step.next), host(nxt), err_msg=f"position {pos}")
        tokens = nxt.clone()
    with pytest.raises(ValueError):
        step.replay(max_length=TINY.context + 1)
