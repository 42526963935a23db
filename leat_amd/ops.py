"""leat's operators on quantized weights (leat/ops.py:18-182) for torch-ROCm tensors: linear,
linears, feed_forward, router, mixture, glu and rms_norm, with the LEAT_KERNELS=ref switch.

Every product goes one of three ways, chosen per call by `_plan`:
- "decode": up to kernels.MATVEC_TOKENS tokens, on the matrix-vector kernels;
- "prefill": more tokens of one sequence, on the matrix-core kernels;
- "reference": LEAT_KERNELS=ref, or a shape neither family takes. The weights are decoded and
  multiplied with f32 activations that are not quantized, as leat's reference ops do. This still
  runs on the GPU: the f32-activation matvec kernel for up to 16 tokens, else the HIP
  dequantizer followed by a library GEMM.
"""

from __future__ import annotations

import os

import torch

from leat_amd import kernels
from leat_amd.quant import NATIVE, QTensor

# gpt-oss's SwiGLU: the sigmoid's slope and the clamp on gate and up (leat/kernels/common.py:21)
OAI_ALPHA, OAI_LIMIT = 1.702, 7.0

Norm = tuple[torch.Tensor, float]


def reference_mode() -> bool:
    """True when LEAT_KERNELS=ref asks for the reference semantics (leat/ops.py:156-157)."""
    return os.environ.get("LEAT_KERNELS") == "ref"


def _plan(x: torch.Tensor, *ws: QTensor) -> str:
    # the kernel family every matrix of the call fits, matrix-vector first (leat/ops.py:31-34)
    if reference_mode():
        return "reference"
    if all(kernels.supports_matvec(x, w) for w in ws):
        return "decode"
    if all(kernels.supports_matmul(x, w) for w in ws):
        return "prefill"
    return "reference"


def linear(x: torch.Tensor, w: QTensor, residual: torch.Tensor | None = None) -> torch.Tensor:
    """x @ w.T, plus `residual` if given (added inside the kernel on the kernel paths)."""
    (out,) = linears(x, w, residual=residual)
    return out


def linears(
    x: torch.Tensor, *ws: QTensor, norm: Norm | None = None, residual: torch.Tensor | None = None
) -> list[torch.Tensor]:
    """x @ w.T for each w, x first RMS-normalized with `norm` = (weight, eps) if given. A residual
    needs a single w. On the kernel paths all products share one int8 quantization of x
    (leat/ops.py:23-38)."""
    plan = _plan(x, *ws)
    if plan == "decode":
        return kernels.matvecs(x, *ws, norm=norm, residual=residual)
    if plan == "prefill":
        return kernels.matmuls(x, *ws, norm=norm, residual=residual)
    source = x if norm is None else rms_norm(x, *norm)
    products = [_reference_product(source, w) for w in ws]
    if residual is not None:
        products = [p + residual for p in products]
    return products


def _reference_product(x: torch.Tensor, w: QTensor) -> torch.Tensor:
    # the reference path's x @ w.dequant(x.dtype).T with x in f32, not quantized
    tokens = x.numel() // x.shape[-1]
    if w.type in NATIVE:  # F32, F16, BF16 weights are their own values
        return x @ w.dequant(x.dtype).T
    if tokens <= kernels.MATVEC_TOKENS or tokens == kernels.FEW_TOKENS:
        return kernels.matvec_f32x(x, w).to(x.dtype)
    return x @ w.dequant(x.dtype).T


def feed_forward(
    x: torch.Tensor, gate: QTensor, up: QTensor, down: QTensor, norm: Norm, kind: str = "silu",
    residual: bool = True,
) -> torch.Tensor:  # fmt: skip
    """A gated MLP on n = rms_norm(x, *norm): glu(kind, n @ gate.T, n @ up.T) @ down.T, plus x
    when `residual` (leat/ops.py:41-55). gate and up of one type and shape go through one kernel
    together; for few tokens that is the matrix-vector GLU kernel, for many the matrix-core
    feed-forward (gate+up, quantize, down) when all three matrices fit it."""
    twins = not reference_mode() and gate.type == up.type and gate.shape == up.shape
    if twins and kernels.supports_matvec(x, gate):
        # down's input has gate's rows as its columns: the decode kernels take it too when its type
        # does; then the whole MLP runs on them (the GLU may quantize its outputs for down itself)
        probe = x.new_empty(*x.shape[:-1], gate.shape[0])
        if kernels.supports_matvec(probe, down):
            return kernels.feed_forward(x, gate, up, down, norm, kind, residual)
        hidden = kernels.swiglu(x, gate, up, norm, kind)
    elif twins and _plan(x, gate, up, down) == "prefill":
        return kernels.feed_forward(x, gate, up, down, norm, kind, residual)
    else:
        g, u = linears(x, gate, up, norm=norm)
        hidden = glu(kind, g, u)
    return linear(hidden, down, residual=x if residual else None)


def router(x: torch.Tensor, norm: Norm, w: QTensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """A mixture's router scores rms_norm(x, *norm) @ w.T, plus `bias` if given (leat/ops.py:80-87):
    one f32 kernel for an F32 router, else the linear product of the normed x."""
    if not reference_mode() and kernels.supports_scores(x, w):
        scores = kernels.scores(x, norm, w)
    else:
        scores = linear(rms_norm(x, *norm), w)
    return scores if bias is None else scores + bias


def mixture(
    x: torch.Tensor, scores: torch.Tensor, gate: QTensor, up: QTensor | None, down: QTensor, used: int,
    norm: Norm, kind: str = "silu", scales: torch.Tensor | None = None, residual: bool = True,
    biases: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None, live: int | None = None,
) -> torch.Tensor:  # fmt: skip
    """A mixture-of-experts MLP (leat/ops.py:90-124) on n = rms_norm(x, *norm), plus x when
    `residual`. Each token runs the gated MLPs of the `used` experts its router `scores`
    (B, T, experts) rank highest, and sums their outputs weighted by the softmax of those scores
    (times `scales[e]` if given).

    The experts are stacks (experts, rows, cols). `biases` = (gate, up, down) biases of shape
    (experts, rows) may be given. Where `up` is None, `gate` holds each expert's gate rows and
    then its up rows. On the kernels, tokens past the first `live` are batch padding: they read
    no experts and their mixture is zero. The reference semantics compute them like any other
    token."""
    if not reference_mode() and used <= kernels.MAX_USED and kernels.supports_mixture(x, gate, up, down):
        return kernels.mixture(x, scores, gate, up, down, used, norm, kind, scales, residual, biases, live)
    dim = x.shape[-1]
    normed = rms_norm(x.float(), *norm).reshape(-1, dim)
    ranked = scores.float().reshape(normed.shape[0], -1).topk(used, dim=-1)
    share = ranked.values.softmax(-1)
    if scales is not None:
        share = share * scales.float()[ranked.indices]
    mixed = torch.zeros_like(normed)
    # every expert some token chose, once, over the tokens that chose it
    for e in ranked.indices.unique().tolist():
        token, slot = (ranked.indices == e).nonzero(as_tuple=True)
        out = _expert_mlp(normed[token], e, gate, up, down, kind, biases)
        mixed.index_add_(0, token, out * share[token, slot].unsqueeze(-1))
    mixed = mixed.reshape(x.shape)
    return x + mixed if residual else mixed


def _expert_mlp(
    n: torch.Tensor, e: int, gate: QTensor, up: QTensor | None, down: QTensor, kind: str,
    biases: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None,
) -> torch.Tensor:  # fmt: skip
    # expert e's gated MLP of the rows n, on its matrices decoded from storage
    g = n @ _expert(gate, e).T
    if up is None:
        g, u = g.chunk(2, dim=-1)
    else:
        u = n @ _expert(up, e).T
    if biases is not None:
        g = g + biases[0][e].float()
        u = u + biases[1][e].float()
    out = glu(kind, g, u) @ _expert(down, e).T
    return out if biases is None else out + biases[2][e].float()


def _expert(stack: QTensor, e: int) -> torch.Tensor:
    # matrix e of a stack (experts, rows, cols), decoded to f32
    per_expert = stack.data.shape[0] // stack.shape[0]
    blocks = stack.data[e * per_expert : (e + 1) * per_expert]
    return QTensor(blocks, stack.type, tuple(stack.shape[1:])).dequant()


def glu(kind: str, g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """The gate/up combination of a gated MLP (leat/ops.py:58-64): silu(g)*u, gelu(g)*u with
    GELU's tanh approximation, or gpt-oss's "oai": gate clamped above and up on both sides at
    OAI_LIMIT, then g*sigmoid(OAI_ALPHA*g)*(u + 1)."""
    if kind == "silu":
        return torch.nn.functional.silu(g) * u
    if kind == "gelu":
        return torch.nn.functional.gelu(g, approximate="tanh") * u
    if kind == "oai":
        gc = torch.clamp(g, max=OAI_LIMIT)
        uc = torch.clamp(u, -OAI_LIMIT, OAI_LIMIT)
        return gc * torch.sigmoid(OAI_ALPHA * gc) * (uc + 1)
    raise ValueError(f"unknown GLU kind {kind!r}")


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) over the last axis, times `weight` if given (leat/ops.py:180-182)."""
    scaled = x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + eps)
    return scaled if weight is None else scaled * weight
