"""The kernels bench.py times, at the shapes it times them, against the CPU oracle.

Config 2's Llama-3-8B layer matrices (q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096 Q4_K, down
4096x14336 Q6_K) at 1, 4, 8 and 16 tokens; the gate+up GLU with its q8 output at 1 token (the
launch that quantizes its own normed input) and 8; and config 4's 512-token prefill GLU on sampled
groups of rows. Weights use the benchmark's synthetic distributions. Each oracle matrix is decoded
once per module into f64 (about 1 GB for the largest shapes).
"""

import functools

import numpy as np
import pytest
import torch

from leat_amd import _lib, kernels, ops
from leat_amd.quant import GGMLType
from oracle import leat_oracle as O
from tests.conftest import assert_close, assert_north_star, gpu, host, make_weights, norm_weight, normal

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = GGMLType.Q4_K, GGMLType.Q6_K

LLAMA = {"q": (Q4_K, 4096, 4096), "kv": (Q4_K, 1024, 4096), "gate": (Q4_K, 14336, 4096), "down": (Q6_K, 4096, 14336)}


@functools.cache
def _matrix(name: str, seed: int = 0):
    # (Weights on the GPU, f64 dense decode) of a benchmark-shaped matrix
    ggml_type, rows, cols = LLAMA[name]
    w = make_weights(ggml_type, rows, cols, np.random.default_rng(100 + seed + 7 * len(name)), synthetic=True)
    return w, O.dequant(int(ggml_type), w.blocks, rows, cols).astype(np.float64)


def _dense_q8(q, d, cols):
    # int8 activations with their group scales, as f64 rows
    return (np.asarray(q).reshape(-1, 32).astype(np.float64) * np.asarray(d, np.float64)[:, None]).reshape(-1, cols)


def _glu_f32(xo, g_dense, u_dense):
    # the GLU of products evaluated in f32, as the reference path sums them: silu(g) * u turns
    # the sums' rounding near g = 0 into an absolute error of |u| times it, which the acceptance
    # bound's absolute floor then allows (conftest.assert_north_star)
    x32 = xo.astype(np.float32)
    return O.glu("silu", x32 @ g_dense.astype(np.float32).T, x32 @ u_dense.astype(np.float32).T)


def _q8_host(t):
    q, d, s = (host(v) for v in t)
    return q.view(np.int8), d, s


@pytest.mark.parametrize("name", list(LLAMA))
@pytest.mark.parametrize("tokens", [1, 4, 8, 16])
def test_llama_layer_shapes(cuda, name, tokens):
    # ops.linear at every config-2 batch size: up to 8 tokens on the decode kernels, 16 on the
    # matrix-core path; against the f64 product of the same q8 activations
    w, dense = _matrix(name)
    rows, cols = dense.shape
    x = normal(np.random.default_rng(tokens), 1, tokens, cols)
    got = host(ops.linear(gpu(x), w.q))[0]
    q, d, _ = O.quantize_q8(x[0])
    want = _dense_q8(q, d, cols) @ dense.T
    f32 = (_dense_q8(q, d, cols).astype(np.float32) @ dense.astype(np.float32).T)
    assert_north_star(got, want, f32)
    assert_close(got, want, 1e-4)


@pytest.mark.parametrize("tokens", [1, 2])
def test_glu_self_quantized_bench_shape(cuda, tokens):
    # leat_glu_matvec_f32 (the B=1 roofline launch): RMSNorm + quantize inside, gate and up
    # 14336x4096, q8 of its outputs for the down product
    gate, g_dense = _matrix("gate", 0)
    up, u_dense = _matrix("gate", 1)
    rows, cols = g_dense.shape
    rng = np.random.default_rng(40 + tokens)
    x = normal(rng, tokens, cols, scale=2.0)
    weight = norm_weight(rng, cols)
    x_gpu, w_gpu = gpu(x), gpu(weight)
    out = torch.empty(tokens * rows, dtype=torch.float32, device=cuda)
    hq = torch.empty(tokens * rows // 4, dtype=torch.int32, device=cuda)
    hd, hs = (torch.empty(tokens * rows // 32, dtype=torch.float32, device=cuda) for _ in range(2))
    _lib.call("leat_glu_matvec_f32", int(Q4_K), gate.q.data.data_ptr(), up.q.data.data_ptr(), rows, cols,
              x_gpu.data_ptr(), tokens, w_gpu.data_ptr(), 1e-5, 0, out.data_ptr(), hq.data_ptr(), hd.data_ptr(),
              hs.data_ptr(), _lib.stream())  # fmt: skip
    got = host(out).reshape(tokens, rows)
    # exactly the activations the standalone quantizer gives: a tight bound
    xq, xd, _ = _q8_host(kernels.quantize_q8(x_gpu, (w_gpu, 1e-5)))
    xs = _dense_q8(xq, xd, cols)
    want = O.glu("silu", xs @ g_dense.T, xs @ u_dense.T)
    assert_close(got, want, 1e-4)
    # the oracle's own f64 RMSNorm: a few int8 activations may move one step
    q, d, _ = O.quantize_q8(O.rms_norm(x, weight, 1e-5))
    xo = _dense_q8(q, d, cols)
    assert_close(got, O.glu("silu", xo @ g_dense.T, xo @ u_dense.T), 1e-3)
    wq, wd, ws = O.quantize_q8(got)
    np.testing.assert_array_equal(host(hq), O.pack_q8(wq))
    np.testing.assert_array_equal(host(hd), wd)
    np.testing.assert_array_equal(host(hs), ws)


@pytest.mark.parametrize("tokens", [3, 8, 16])
def test_glu_q8_bench_shape(cuda, tokens):
    # leat_glu_matvec_q8 (the B=8 and B=16 launches: the matrix-core tile kernel writing its
    # outputs' q8)
    gate, g_dense = _matrix("gate", 0)
    up, u_dense = _matrix("gate", 1)
    rows, cols = g_dense.shape
    x = normal(np.random.default_rng(50 + tokens), tokens, cols, scale=2.0)
    xq, xd, xs = kernels.quantize_q8(gpu(x))
    out = torch.empty(tokens * rows, dtype=torch.float32, device=cuda)
    hq = torch.empty(tokens * rows // 4, dtype=torch.int32, device=cuda)
    hd, hs = (torch.empty(tokens * rows // 32, dtype=torch.float32, device=cuda) for _ in range(2))
    _lib.call("leat_glu_matvec_q8", int(Q4_K), gate.q.data.data_ptr(), up.q.data.data_ptr(), rows, cols,
              xq.data_ptr(), xd.data_ptr(), xs.data_ptr(), tokens, 0, out.data_ptr(), hq.data_ptr(), hd.data_ptr(),
              hs.data_ptr(), _lib.stream())  # fmt: skip
    got = host(out).reshape(tokens, rows)
    q, d, _ = O.quantize_q8(x)
    xo = _dense_q8(q, d, cols)
    want = O.glu("silu", xo @ g_dense.T, xo @ u_dense.T)
    assert_north_star(got, want, _glu_f32(xo, g_dense, u_dense))
    assert_close(got, want, 1e-4)
    wq, wd, ws = O.quantize_q8(got)
    np.testing.assert_array_equal(host(hq), O.pack_q8(wq))
    np.testing.assert_array_equal(host(hd), wd)
    np.testing.assert_array_equal(host(hs), ws)


def test_prefill_glu_q8_bench_shape(cuda):
    # config 4's gate+up launch, 512 tokens: f32 outputs on sampled groups of 32 rows (first,
    # last, and tiles between) against the oracle, and the q8 output exactly the quantizer of the
    # f32 output over every row
    gate, g_dense = _matrix("gate", 0)
    up, u_dense = _matrix("gate", 1)
    rows, cols = g_dense.shape
    tokens = 512
    x = normal(np.random.default_rng(60), tokens, cols)
    xq, xd, xs = kernels.quantize_q8(gpu(x))
    out = torch.empty(tokens * rows, dtype=torch.float32, device=cuda)
    hq = torch.empty(tokens * rows // 4, dtype=torch.int32, device=cuda)
    hd, hs = (torch.empty(tokens * rows // 32, dtype=torch.float32, device=cuda) for _ in range(2))
    _lib.call("leat_glu_matmul_q8", int(Q4_K), gate.q.data.data_ptr(), up.q.data.data_ptr(), rows, cols,
              xq.data_ptr(), xd.data_ptr(), xs.data_ptr(), tokens, 0, out.data_ptr(), hq.data_ptr(), hd.data_ptr(),
              hs.data_ptr(), None, 0, _lib.stream())  # fmt: skip
    got = host(out).reshape(tokens, rows)
    q, d, _ = O.quantize_q8(x)
    xo = _dense_q8(q, d, cols)
    sample = np.concatenate([np.arange(32 * g, 32 * g + 32) for g in (0, 1, 2, 3, 100, 223, 224, 301, 446, 447)])
    want = O.glu("silu", xo @ g_dense[sample].T, xo @ u_dense[sample].T)
    assert_north_star(got[:, sample], want, _glu_f32(xo, g_dense[sample], u_dense[sample]))
    assert_close(got[:, sample], want, 1e-4)
    wq, wd, ws = O.quantize_q8(got)
    np.testing.assert_array_equal(host(hq), O.pack_q8(wq))
    np.testing.assert_array_equal(host(hd), wd)
    np.testing.assert_array_equal(host(hs), ws)


def test_prefill_down_bench_shape(cuda):
    # config 4's Q6_K down product with its residual, 512 tokens, on sampled rows
    down, dense = _matrix("down")
    rows, cols = dense.shape
    tokens = 512
    rng = np.random.default_rng(61)
    h = normal(rng, tokens, cols)
    residual = normal(rng, tokens, rows)
    got = host(kernels.matmuls(gpu(h[None]), down.q, residual=gpu(residual[None]))[0])[0]
    q, d, _ = O.quantize_q8(h)
    sample = np.r_[0:64, 1984:2112, 4032:4096]
    want = _dense_q8(q, d, cols) @ dense[sample].T + residual[:, sample]
    assert_close(got[:, sample], want, 1e-4)


def test_output_head_shape(cuda):
    # config 3's Q6_K output head (128256 x 4096) with the final RMSNorm, as the decode step runs
    # it: a launch past SELF_QUANTIZED_ROWS quantizes x once and takes the q8-input product, which
    # must equal the one-launch f32 path bit for bit; sampled rows against the oracle
    vocab, cols = 128256, 4096
    rng = np.random.default_rng(77)
    blocks = O.matrix_blocks(int(Q6_K), vocab, cols, rng, synthetic=True, scale=1e-3)
    from leat_amd.quant import from_blocks

    head = from_blocks(blocks, Q6_K, (vocab, cols))
    x = normal(rng, 1, cols, scale=2.0)
    weight = norm_weight(rng, cols)
    x_gpu, w_gpu = gpu(x), gpu(weight)
    assert vocab > kernels.SELF_QUANTIZED_ROWS
    got = host(kernels.matvecs(x_gpu, head, norm=(w_gpu, 1e-5))[0])[0]
    one = torch.empty(vocab, dtype=torch.float32, device=cuda)
    _lib.call("leat_matvec_f32", int(Q6_K), head.data.data_ptr(), vocab, cols, x_gpu.data_ptr(), 1, w_gpu.data_ptr(),
              1e-5, None, one.data_ptr(), _lib.stream())  # fmt: skip
    np.testing.assert_array_equal(got, host(one))
    sample = np.sort(rng.choice(vocab, 512, replace=False))
    per_row = blocks.reshape(vocab, -1, blocks.shape[-1])[sample].reshape(-1, blocks.shape[-1])
    dense = O.dequant(int(Q6_K), per_row, len(sample), cols).astype(np.float64)
    xq, xd, _ = _q8_host(kernels.quantize_q8(x_gpu, (w_gpu, 1e-5)))
    assert_close(got[sample], (_dense_q8(xq, xd, cols) @ dense.T)[0], 1e-4)
    q, d, _ = O.quantize_q8(O.rms_norm(x, weight, 1e-5))
    assert_close(got[sample], (_dense_q8(q, d, cols) @ dense.T)[0], 1e-3)
