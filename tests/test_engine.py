"""Batched decoding (leat_amd/engine.py, after leat/engine.py:124-189, 546-583): the batch sizes
that get a graph, which of them take padding, and how a step's sequences split into batches (on
the CPU); then on the GPU, sequences decoded together in padded batches against each decoded
alone, and the padding rows leaving every sequence's cache as it was."""

import numpy as np
import pytest

from leat_amd.engine import BATCH, batch_sizes, padded_sizes, plan


def test_batch_sizes_and_padding():
    assert BATCH == 8
    assert batch_sizes(1) == [1] and padded_sizes([1]) == set()
    assert batch_sizes(3) == [1, 2, 3] and padded_sizes(batch_sizes(3)) == set()
    assert batch_sizes(4) == [1, 2, 4] and padded_sizes(batch_sizes(4)) == {4}
    assert batch_sizes(6) == [1, 2, 4, 6] and padded_sizes(batch_sizes(6)) == {4, 6}
    assert batch_sizes(8) == [1, 2, 4, 8] and padded_sizes(batch_sizes(8)) == {4, 8}
    assert batch_sizes(32) == [1, 2, 4, 8]  # at most BATCH a step
    with pytest.raises(StopIteration):  # no size holds more than the slots
        plan(3, [1, 2])


def test_plan_pads_3_to_4_and_5_to_7_to_8():
    sizes = batch_sizes(16)
    assert [plan(k, sizes) for k in (1, 2, 3, 4)] == [[(0, 1)], [(0, 2)], [(0, 4)], [(0, 4)]]
    assert all(plan(k, sizes) == [(0, 8)] for k in (5, 6, 7, 8))
    assert plan(11, sizes) == [(0, 8), (8, 4)]
    assert plan(16, sizes) == [(0, 8), (8, 8)]


@pytest.mark.gpu
def test_batched_decode_matches_alone(cuda):
    import torch

    from leat_amd.engine import Engine
    from leat_amd.model import LlamaConfig, synthetic
    from tests.conftest import host

    cfg = LlamaConfig(dim=512, layers=2, heads=8, kv_heads=2, head_dim=128, ffn=1024, vocab=1000, context=128,
                      rope_theta=10000.0, rope_scaling=None)  # fmt: skip
    weights = synthetic(cfg, seed=11)
    prompts = [[5, 6, 7], list(range(100, 112)), [42], [9, 8, 7, 6, 5], [1, 2], [300, 301, 302, 303, 304, 305, 306]]
    steps = 5
    # each alone: one slot, batches of 1
    alone = []
    for p in prompts:
        e = Engine(cfg, weights, slots=1)
        s = e.start(p)
        for _ in range(steps):
            e.decode([s])
        alone.append(s.tokens)
    # together: 8 slots; 6 sequences run in the padded graph of 8, then 3 in that of 4
    e = Engine(cfg, weights, slots=8)
    assert e.padded == {4, 8} and e.model.config.slots == 9
    seqs = [e.start(p) for p in prompts]
    for _ in range(steps):
        e.decode(seqs)
    for _ in range(2):
        e.decode(seqs[:3])
    for s, want in zip(seqs, alone, strict=True):
        assert s.tokens[: len(want)] == want
    assert sorted(e._graphs) == [4, 8]
    # the spare slot took the padding; every sequence's slot holds exactly its own positions
    for cache in e.model.cache:
        c = host(cache)
        assert np.abs(c[:, e.spare, :, 0]).sum() > 0 and not c[:, e.spare, :, 1:].any()
        for s in seqs:
            assert not c[:, s.slot, :, s.cached :].any()


@pytest.mark.gpu
def test_engine_decode_across_length_buckets(cuda):
    # a sequence whose decode steps cross 128 positions: the engine replays the short-context
    # graph, then the context's; every token that of eager steps sized for the whole context
    import torch

    from leat_amd.engine import Engine
    from leat_amd.model import LlamaConfig, Model, synthetic

    cfg = LlamaConfig(dim=512, layers=2, heads=8, kv_heads=2, head_dim=128, ffn=1024, vocab=1000, context=256,
                      rope_theta=10000.0, rope_scaling=None)  # fmt: skip
    weights = synthetic(cfg, seed=12)
    prompt = [int(t) for t in np.random.default_rng(12).integers(0, cfg.vocab, 120)]
    steps = 16
    e = Engine(cfg, weights, slots=1)
    s = e.start(prompt)
    for _ in range(steps):
        e.decode([s])
    assert e._graphs[1].buckets == (128, 256)
    model = Model(LlamaConfig(**{**cfg.__dict__, "slots": 1}), weights)
    one = torch.zeros(1, dtype=torch.int32, device=cuda)
    ids = torch.tensor(prompt, dtype=torch.int32, device=cuda)
    nxt = model.step(ids, one.expand(len(prompt)).contiguous(), torch.arange(len(prompt), dtype=torch.int32, device=cuda),
                     last=True)  # fmt: skip
    tokens = list(prompt) + [int(nxt[-1])]
    for pos in range(len(prompt), len(prompt) + steps):
        nxt = model.step(torch.tensor([tokens[-1]], dtype=torch.int32, device=cuda), one,
                         torch.tensor([pos], dtype=torch.int32, device=cuda))  # fmt: skip
        tokens.append(int(nxt[0]))
    assert s.tokens == tokens
