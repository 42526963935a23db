"""The storage types beyond Q4_K, Q6_K and Q8_0 (leat/quant.py:94-231, leat/kernels/matvec.py:
184-303) on a gfx950 GPU against the oracle: the dequantizer bit for bit for all 13 types leat
decodes, the int32 group sums of the 11 the decode tasks take, their decode and prefill products,
and the LEAT_KERNELS=ref product on every one."""

import numpy as np
import pytest

from leat_amd import kernels, ops
from leat_amd.quant import GGMLType, MATVEC_TYPES
from oracle import leat_oracle as O
from tests.conftest import assert_close, assert_north_star, gpu, host, make_weights, normal

pytestmark = pytest.mark.gpu
ALL = [GGMLType(t) for t in O.NAMES]
NEW = [t for t in MATVEC_TYPES if t not in (GGMLType.Q4_K, GGMLType.Q6_K, GGMLType.Q8_0)]


def _cols(t):
    return 2048 if O.BLOCK[int(t)][0] == 256 else 2112  # 2112: 33 pairs of blocks, a partial wave turn


@pytest.mark.parametrize("ggml_type", ALL, ids=lambda t: t.name)
def test_dequantize_all_types(cuda, ggml_type):
    rng = np.random.default_rng(70)
    rows, cols = 48, _cols(ggml_type)
    w = make_weights(ggml_type, rows, cols, rng)
    got = host(w.q.dequant()).reshape(-1)
    want = O.dequant_blocks(int(ggml_type), w.blocks).reshape(-1)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("ggml_type", NEW, ids=lambda t: t.name)
@pytest.mark.parametrize("tokens", [1, 3, 8])
def test_group_sums_new_types(cuda, ggml_type, tokens):
    rng = np.random.default_rng(71)
    rows, cols = 40, _cols(ggml_type)
    w = make_weights(ggml_type, rows, cols, rng)
    x = normal(rng, tokens, cols, scale=3.0)
    xq, _, _ = kernels.quantize_q8(gpu(x))
    got = host(kernels.group_dots(xq, w.q, tokens))
    q, _, _ = O.quantize_q8(x)
    np.testing.assert_array_equal(got, O.group_dots(int(ggml_type), w.blocks, rows, cols, q))


@pytest.mark.parametrize("ggml_type", NEW, ids=lambda t: t.name)
@pytest.mark.parametrize("tokens", [1, 5, 8])
def test_matvec_new_types(cuda, ggml_type, tokens):
    # leat's matvec shapes (tests/test_kernels.py:106-116), rows of whole pairs of blocks
    rng = np.random.default_rng(72)
    for rows, cols in ((64, 4096), (24, 2816 if O.BLOCK[int(ggml_type)][0] == 32 else 2816 + 256)):
        w = make_weights(ggml_type, rows, cols, rng)
        x = normal(rng, 1, tokens, cols)
        assert kernels.supports_matvec(gpu(x), w.q)
        got = host(ops.linear(gpu(x), w.q))[0]
        want = w.product(x[0])
        assert_close(got, want, 1e-4)
        assert_north_star(got, want, O.reference_matmul_f32(x[0], w.blocks, int(ggml_type)))


@pytest.mark.parametrize("ggml_type", NEW, ids=lambda t: t.name)
def test_swiglu_and_prefill_new_types(cuda, ggml_type):
    # the gated product at 4 tokens, and 20- and 70-token prefill products (8 tokens a launch)
    rng = np.random.default_rng(73)
    cols = 1024
    gate, up = make_weights(ggml_type, 64, cols, rng), make_weights(ggml_type, 64, cols, rng)
    x = normal(rng, 1, 4, cols, scale=3.0)
    got = host(kernels.swiglu(gpu(x), gate.q, up.q))[0]
    assert_close(got, O.glu("silu", gate.product(x[0]), up.product(x[0])), 1e-4)
    for tokens in (20, 70):
        x = normal(rng, 1, tokens, cols)
        residual = normal(rng, 1, tokens, 64)
        assert kernels.supports_matmul(gpu(x), gate.q)
        got = host(ops.linear(gpu(x), gate.q, residual=gpu(residual)))[0]
        assert_close(got, gate.product(x[0]) + residual[0], 1e-4)


@pytest.mark.parametrize("ggml_type", ALL, ids=lambda t: t.name)
def test_reference_switch_all_types(cuda, monkeypatch, ggml_type):
    # LEAT_KERNELS=ref: f32 activations against x @ dequant(W).T in f64, every type leat decodes
    rng = np.random.default_rng(74)
    rows, cols = 40, _cols(ggml_type)
    w = make_weights(ggml_type, rows, cols, rng)
    x = normal(rng, 1, 3, cols)
    monkeypatch.setenv("LEAT_KERNELS", "ref")
    got = host(ops.linear(gpu(x), w.q))[0]
    assert_close(got, O.ref_linear(x[0], w.blocks, int(ggml_type), rows, cols), 1e-5)
