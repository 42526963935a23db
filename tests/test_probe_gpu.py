"""The measurement probes bench.py reports beside the published peaks (leat_probe_read,
leat_probe_mfma_i8): each must do all its work, which their results show exactly."""

import numpy as np
import pytest
import torch

from leat_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("chunks,workgroups", [(1, 1), (65_539, 7), (1 << 18, 1024)])
def test_probe_read_sums_every_word(cuda, chunks, workgroups):
    # every 32-bit word summed modulo 2^32, whatever the chunk count against the grid
    rng = np.random.default_rng(chunks)
    words = rng.integers(0, 1 << 32, size=4 * chunks, dtype=np.uint64).astype(np.uint32)
    data = torch.from_numpy(words.view(np.int32)).to(cuda)
    sink = torch.empty(workgroups, dtype=torch.int32, device=cuda)
    _lib.call("leat_probe_read", data.data_ptr(), 16 * chunks, sink.data_ptr(), workgroups, _lib.stream())
    got = int(sink.cpu().numpy().view(np.uint32).astype(np.uint64).sum()) % (1 << 32)
    assert got == int(words.astype(np.uint64).sum()) % (1 << 32)


def test_probe_mfma_runs_every_product(cuda):
    # all-ones operands: each v_mfma_i32_32x32x32_i8 adds 32 to every element of its accumulator
    iters, workgroups = 37, 9
    sink = torch.full((4 * workgroups,), -1, dtype=torch.int32, device=cuda)
    _lib.call("leat_probe_mfma_i8", iters, workgroups, sink.data_ptr(), _lib.stream())
    assert (sink.cpu() == 128 * iters).all()


def test_probe_arguments_checked(cuda):
    data = torch.zeros(16, dtype=torch.int32, device=cuda)
    sink = torch.empty(4, dtype=torch.int32, device=cuda)
    with pytest.raises(_lib.LeatError, match="16-byte"):
        _lib.call("leat_probe_read", data.data_ptr(), 24, sink.data_ptr(), 1, _lib.stream())
    with pytest.raises(_lib.LeatError, match="rounds"):
        _lib.call("leat_probe_mfma_i8", 0, 1, sink.data_ptr(), _lib.stream())
