"""leat_matmul_noalloc (include/leatmi.h): the split prefill product with its partial sums in the
library's own device array, against leat_matmul with a caller workspace, bit for bit: two calls
in a row, the second smaller (the array keeps the first call's sums), then a product whose split
needs more than the array holds, which must be refused."""

import numpy as np
import pytest
import torch

from leat_amd import _lib, kernels
from leat_amd.quant import GGMLType
from tests.conftest import gpu, host, make_weights, normal

pytestmark = pytest.mark.gpu


def _with_workspace(w, q8, tokens, residual):
    xq, xd, xs = q8
    rows, cols = w.q.shape
    out = torch.empty(tokens * rows, dtype=torch.float32, device=xq.device)
    size = _lib.workspace_bytes(w.type, rows, cols, tokens, False)
    assert size > 0  # the product splits on 256 compute units
    ws = torch.empty(size, dtype=torch.uint8, device=xq.device)
    _lib.call("leat_matmul", int(w.type), w.q.data.data_ptr(), rows, cols, xq.data_ptr(), xd.data_ptr(), xs.data_ptr(),
              tokens, _lib.ptr(residual), out.data_ptr(), ws.data_ptr(), size, _lib.stream())  # fmt: skip
    return host(out)


def _no_alloc(w, q8, tokens, residual):
    xq, xd, xs = q8
    rows, cols = w.q.shape
    out = torch.empty(tokens * rows, dtype=torch.float32, device=xq.device)
    _lib.call("leat_matmul_noalloc", int(w.type), w.q.data.data_ptr(), rows, cols, xq.data_ptr(), xd.data_ptr(),
              xs.data_ptr(), tokens, _lib.ptr(residual), out.data_ptr(), _lib.stream())  # fmt: skip
    return host(out)


# (type, rows, cols, token counts of the two calls): Llama-3-8B's down and o shapes
@pytest.mark.parametrize("ggml_type, rows, cols, calls", [(GGMLType.Q6_K, 4096, 14336, (100, 40)),
                                                          (GGMLType.Q4_K, 4096, 4096, (64, 20))])  # fmt: skip
def test_no_alloc_matches_workspace(cuda, ggml_type, rows, cols, calls):
    rng = np.random.default_rng(200)
    w = make_weights(ggml_type, rows, cols, rng, synthetic=True)
    for tokens in calls:  # the second call smaller: stale sums of the first stay in the array
        x = normal(rng, tokens, cols)
        residual = gpu(normal(rng, tokens, rows))
        q8 = kernels.quantize_q8(gpu(x))
        want = _with_workspace(w, q8, tokens, residual)
        got = _no_alloc(w, q8, tokens, residual)
        np.testing.assert_array_equal(got, want)


def test_no_alloc_refuses_past_its_array(cuda):
    # 28672 rows of Q4_K at 64 tokens split into 224 tiles x 2 chunks of 32 KiB: 14.7 MB > 8 MiB
    rows, cols, tokens = 28672, 4096, 64
    assert _lib.workspace_bytes(GGMLType.Q4_K, rows, cols, tokens, False) > 8 << 20
    w = torch.zeros(rows * cols // 256 * 144, dtype=torch.uint8, device=cuda)
    xq = torch.zeros(tokens * cols // 4, dtype=torch.int32, device=cuda)
    xd = torch.zeros(tokens * cols // 32, dtype=torch.float32, device=cuda)
    out = torch.empty(tokens * rows, dtype=torch.float32, device=cuda)
    with pytest.raises(_lib.LeatError, match="no-allocation"):
        _lib.call("leat_matmul_noalloc", int(GGMLType.Q4_K), w.data_ptr(), rows, cols, xq.data_ptr(), xd.data_ptr(),
                  xd.data_ptr(), tokens, None, out.data_ptr(), _lib.stream())  # fmt: skip
