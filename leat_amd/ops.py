"""leat's operators on quantized weights (leat/ops.py:18-182) for torch-ROCm tensors: linear,
linears, feed_forward, router, mixture, glu and rms_norm, and the decode step's embedding, rotate,
attention and argmax (leat/ops.py:166-376, 496-500), with the LEAT_KERNELS=ref switch.

Every product goes one of three ways, chosen per call by `_plan`:
- "decode": up to kernels.MATVEC_TOKENS tokens, on the matrix-vector kernels;
- "prefill": more tokens of one sequence, on the matrix-core kernels;
- "reference": LEAT_KERNELS=ref, or a shape neither family takes. The weights are decoded and
  multiplied with f32 activations that are not quantized, as leat's reference ops do. This still
  runs on the GPU: the f32-activation matvec kernel for up to 16 tokens, else the HIP
  dequantizer followed by a library GEMM.
"""

from __future__ import annotations

import math
import os
from dataclasses import dataclass

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


# ------------------------------------------------------------------ the decode step around them


def embedding(tokens: torch.Tensor, w: QTensor) -> torch.Tensor:
    """The rows of w (vocab, dim) of token ids, decoded: (…, dim) f32 (leat/ops.py:166-178)."""
    if not reference_mode() and kernels.supports_embedding(w):
        return kernels.embedding(tokens, w)
    vocab, dim = w.shape
    ids = tokens.reshape(-1).long().to(w.data.device)
    if w.type in NATIVE:
        return w.data.reshape(vocab, dim)[ids].float().view(*tokens.shape, dim)
    rows = w.data.reshape(vocab, -1)[ids].reshape(-1, w.data.shape[-1]).contiguous()
    return QTensor(rows, w.type, (ids.numel(), dim)).dequant().view(*tokens.shape, dim)


@dataclass(frozen=True)
class Span:
    """`length` consecutive tokens of one sequence from position `start` of cache slot `slot`
    (leat/ops.py:201-209). The kernels here take spans of one token: a decode step's rows."""

    slot: int
    start: int
    length: int = 1


def _span_rows(spans: list[Span]) -> tuple[list[int], list[int]]:
    # each token's slot and position
    rows = [(s.slot, s.start + i) for s in spans for i in range(s.length)]
    return [r[0] for r in rows], [r[1] for r in rows]


def rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, halves: bool) -> torch.Tensor:
    """The first R dimensions of x (B, H, T, D) turned by RoPE, adjacent pairs or with `halves`
    dimensions i and i + R/2; cos, sin (T, R/2) (leat/ops.py:185-198)."""
    rotated = 2 * cos.shape[-1]
    x, rest = x[..., :rotated], x[..., rotated:]
    if halves:
        x0, x1 = x.chunk(2, dim=-1)
        out = torch.cat([x0 * cos - x1 * sin, x0 * sin + x1 * cos], dim=-1)
    else:
        pairs = x.reshape(*x.shape[:-1], -1, 2)
        x0, x1 = pairs[..., 0], pairs[..., 1]
        out = torch.stack([x0 * cos - x1 * sin, x0 * sin + x1 * cos], dim=-1).flatten(-2)
    return out if rest.shape[-1] == 0 else torch.cat([out, rest], dim=-1)


def rotate(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cache: torch.Tensor, spans: list[Span] | None,
    rope: tuple[tuple[torch.Tensor, torch.Tensor], int] | None, halves: bool, slots=None, positions=None,
) -> tuple[torch.Tensor, torch.Tensor]:  # fmt: skip
    """q (1, T, H, D), k and v (1, T, KV_H, D), the spans' tokens in turn: the first R dimensions of
    q and k turned by RoPE at the tokens' positions, k and v stored in their slots of the f16 cache
    (2, slots, KV_H, positions, D) (leat/ops.py:212-276). `slots` and `positions` (device tensors,
    a token each) may replace the spans, as a captured decode step passes them. Returns q
    (1, H, T, D) f32 and the cache."""
    if slots is None:
        slots, positions = _span_rows(spans)
    if not reference_mode() and kernels.supports_rotate(q, cache):
        return kernels.rotate(q, k, v, cache, slots, positions, rope, halves)
    # the reference semantics token by token, in f32 torch ops
    slot_list = slots.tolist() if isinstance(slots, torch.Tensor) else list(slots)
    pos_list = positions.tolist() if isinstance(positions, torch.Tensor) else list(positions)
    q, k, v = (t.float() for t in (q, k, v))
    outs = []
    for t, (slot, pos) in enumerate(zip(slot_list, pos_list, strict=True)):
        qt, kt = q[:, t : t + 1].transpose(1, 2), k[:, t : t + 1].transpose(1, 2)
        if rope is not None:
            cos, sin = (table[pos : pos + 1].float() for table in rope[0])
            qt, kt = rotary(qt, cos, sin, halves), rotary(kt, cos, sin, halves)
        cache[0, slot, :, pos] = kt[0, :, 0].to(cache.dtype)
        cache[1, slot, :, pos] = v[0, t].to(cache.dtype)
        outs.append(qt)
    return torch.cat(outs, dim=2), cache


def qkv_rotate(
    x: torch.Tensor, wq: QTensor, wk: QTensor, wv: QTensor, norm: tuple[torch.Tensor, float] | None,
    cache: torch.Tensor, spans: list[Span] | None, rope: tuple[tuple[torch.Tensor, torch.Tensor], int] | None,
    halves: bool, slots=None, positions=None,
) -> torch.Tensor:  # fmt: skip
    """An attention layer's inputs: linears(x, wq, wk, wv, norm=norm) then rotate() of the three
    into the cache (leat/model.py:397-401: the q, k, v products, RoPE and the KV store), in one
    launch where the kernels take the shapes, with the same results. Returns q rotated (1, H, T, D)
    f32."""
    if slots is None:
        slots, positions = _span_rows(spans)
    if not reference_mode() and kernels.supports_qkv_rotate(x, wq, wk, wv, cache, halves, norm):
        return kernels.qkv_rotate(x, wq, wk, wv, norm, cache, slots, positions, rope)
    dim, kv_heads = cache.shape[-1], cache.shape[2]
    T = x.shape[-2]
    q, k, v = linears(x, wq, wk, wv, norm=norm)
    q_rot, _ = rotate(q.reshape(1, T, wq.shape[0] // dim, dim), k.reshape(1, T, kv_heads, dim),
                      v.reshape(1, T, kv_heads, dim), cache, None, rope, halves, slots, positions)  # fmt: skip
    return q_rot


def attention(
    q: torch.Tensor, cache: torch.Tensor, spans: list[Span] | None, scale: float, slots=None, lengths=None,
    max_length: int | None = None, workspace: torch.Tensor | None = None,
) -> torch.Tensor:  # fmt: skip
    """q (1, H, T, D), the spans' tokens in turn, each token attending causally over its slot's
    positions up to its own, scores q.k * scale (leat/ops.py:305-339). `slots` and `lengths`
    (device tensors, a row each) may replace the spans; `workspace` (kernels.attention_workspace)
    is reused by the kernel path. Returns (1, T, H * D) f32."""
    if slots is None:
        slots, positions = _span_rows(spans)
        lengths = [p + 1 for p in positions]
    if not reference_mode() and kernels.supports_attention(q, cache):
        return kernels.attention(q, cache, slots, lengths, scale, max_length, workspace)
    slot_list = slots.tolist() if isinstance(slots, torch.Tensor) else list(slots)
    length_list = lengths.tolist() if isinstance(lengths, torch.Tensor) else list(lengths)
    _, heads, _, dim = q.shape
    group = heads // cache.shape[2]
    outs = []
    for t, (slot, length) in enumerate(zip(slot_list, length_list, strict=True)):
        keys = cache[0, slot, :, :length].float().repeat_interleave(group, dim=0).contiguous()
        values = cache[1, slot, :, :length].float().repeat_interleave(group, dim=0).contiguous()
        scores = torch.matmul(q[0, :, t : t + 1].float(), keys.transpose(-1, -2).contiguous()) * scale
        outs.append(torch.matmul(scores.softmax(-1), values).reshape(1, heads * dim))
    return torch.stack(outs, dim=1)


def attention_linear(
    q: torch.Tensor, cache: torch.Tensor, spans: list[Span] | None, scale: float, w: QTensor,
    residual: torch.Tensor | None = None, slots=None, lengths=None, max_length: int | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:  # fmt: skip
    """linear(attention(q, cache, ...), w, residual): an attention layer's output product
    (leat/model.py:402-403), with the same results. On the kernel paths the attention kernels
    write the q8 of their output themselves (kernels.attention_q8) and the product takes it as
    it is, instead of quantizing the output again. Returns (1, T, w rows) f32."""
    if slots is None:
        slots, positions = _span_rows(spans)
        lengths = [p + 1 for p in positions]
    att_shape = (1, q.shape[2], q.shape[1] * q.shape[3])
    # a stand-in of the attention output's shape and device, for the product's plan
    stand_in = q.new_empty((1, 1, 1)).expand(att_shape)
    if not reference_mode() and kernels.supports_attention(q, cache) and _plan(stand_in, w) == "decode":
        _, q8 = kernels.attention_q8(q, cache, slots, lengths, scale, max_length, workspace)
        (out,) = kernels.matvecs_quantized(q8, att_shape[1], att_shape[2], w, residual=residual)
        return out.view(1, att_shape[1], w.shape[0])
    att = attention(q, cache, None, scale, slots, lengths, max_length, workspace)
    return linear(att, w, residual=residual)


def argmax(x: torch.Tensor) -> torch.Tensor:
    """Each row's index of its largest value, the first one among equal values: (B, V) -> (B, 1)
    int32 (leat/ops.py:496-500)."""
    if not reference_mode() and kernels.supports_argmax(x):
        return kernels.argmax(x)
    return x.float().nan_to_num(nan=-math.inf).argmax(-1, keepdim=True).to(torch.int32)
