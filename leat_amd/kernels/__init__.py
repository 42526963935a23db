"""The kernel families leat's ops call (leat/kernels/__init__.py:9-45), implemented by the gfx950
HIP kernels of libleatmi.so and called on torch-ROCm tensors.

The families are decode matvec, activation quantizer, prefill matmul, and routing plus expert
products. Each keeps leat's function names, arguments and results, and has a `supports_*`
predicate. A predicate accepts exactly the shapes leat's predicate accepts, and also requires
the tensors to live on a gfx950 GPU. leat_amd.ops consults the predicates to choose between
these kernels and the reference semantics.
"""

from __future__ import annotations

import ctypes

import torch

from leat_amd import _lib
from leat_amd.kernels.attention import (
    argmax,
    attention,
    attention_q8,
    attention_workspace,
    embedding,
    rotate,
    supports_argmax,
    supports_attention,
    supports_embedding,
    supports_rotate,
)
from leat_amd.quant import BLOCK, KERNEL_TYPES, MATVEC_TYPES, GGMLType, QTensor

GROUP = 32  # int8 activations sharing one scale (leat/kernels/common.py:20)
MATVEC_TOKENS = 8  # the most tokens the decode kernels take (leat/kernels/matvec.py:36)
FEW_TOKENS = 16  # leat's tile height for short prompts (leat/kernels/matmul.py:54)
GLU_KINDS = {"silu": 0, "gelu": 1, "oai": 2}
MAX_USED = 64  # the most experts a token may take on the expert kernels (include/leatmi.h)
MAX_PAIRS = 65535  # (token, slot) pairs of one expert launch: longer prompts run in chunks of tokens

Norm = tuple[torch.Tensor, float]
Q8 = tuple[torch.Tensor, torch.Tensor, torch.Tensor]


def _on_gfx950(x: torch.Tensor) -> bool:
    if not x.is_cuda:
        return False
    index = torch.cuda.current_device() if x.device.index is None else x.device.index
    return _lib.device_ok(index)


def _rows_of(x: torch.Tensor) -> int:
    # tokens in x (…, cols)
    return x.numel() // x.shape[-1]


def _f32(x: torch.Tensor) -> torch.Tensor:
    return x.float().contiguous()


def _aligned(t: torch.Tensor) -> torch.Tensor:
    # t contiguous and 16-byte aligned (a view into a mapped file may be neither)
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _blocks(w: QTensor) -> int:
    # the device address of a weight's GGUF blocks
    if w.data.dtype != torch.uint8 or not w.data.is_contiguous():
        raise _lib.LeatError("a QTensor's blocks must be one contiguous uint8 tensor")
    return w.data.data_ptr()


def _q8_buffers(count: int, n: int, device: torch.device) -> Q8:
    words = torch.empty(count * n // 4, dtype=torch.int32, device=device)
    scales = torch.empty(count * n // GROUP, dtype=torch.float32, device=device)
    return words, scales, torch.empty_like(scales)


# tokens up to which the decode kernels quantize their own f32 input (include/leatmi.h
# leat_matvecs_f32): bit-identical to quantize_q8 followed by the product, one launch fewer
SELF_QUANTIZED_TOKENS = 2
# ... in launches of at most this many rows: every workgroup of such a launch normalizes and
# quantizes x again, which past about 32768 rows (an output head: 128256) costs more than one
# quantizer launch (130 against 94 us for a 128256 x 4096 Q6_K head on MI355X)
SELF_QUANTIZED_ROWS = 32768


def _self_quantized(ggml_type: GGMLType, cols: int, tokens: int) -> bool:
    # the shapes the row-streaming kernels take with f32 input (rows_fits in rows.hip)
    if not 0 < tokens <= SELF_QUANTIZED_TOKENS:
        return False
    if ggml_type == GGMLType.Q4_K:
        return cols % 256 == 0 and cols <= 8192
    if ggml_type == GGMLType.Q8_0:
        return cols % 64 == 0 and cols <= 8192
    if ggml_type == GGMLType.Q6_K:
        return cols % 512 == 0 and cols <= 8192
    return False


def _aligned16(*ts: torch.Tensor | None) -> bool:
    # the f32-input kernels read x and the norm weight in 16-byte loads
    return all(t is None or t.data_ptr() % 16 == 0 for t in ts)


def _norm_args(norm: Norm | None) -> tuple[torch.Tensor | None, float]:
    return (None, 0.0) if norm is None else (_f32(norm[0]), float(norm[1]))


# ------------------------------------------------------------------------------ quantizer


def quantize_q8(x: torch.Tensor, norm: Norm | None = None, rows: int | None = None) -> Q8:
    """int8 activations for the products (leat/kernels/quantize.py:92-109). Each row of x (R, n)
    is RMS-normalized with `norm` = (weight, eps) if given, then cut into groups of 32. A group
    gets d = max|value|/127, its values roundf(value/d), and s = d·Σ of those values. With `rows`,
    only that many leading rows are quantized.

    Returns (words, d, s): the int8 values packed four to an int32 word, value 4w+i in byte i of
    word w, and the per-group d and s. Each is one flat tensor, row after row."""
    _lib.require_device(x)
    count, n = x.shape
    src = _aligned(_f32(x))  # the quantizer reads x and the weight in 16-byte loads
    q, d, s = _q8_buffers(count, n, src.device)
    weight, eps = (None, 0.0) if norm is None else (_aligned(_f32(norm[0])), float(norm[1]))
    done = count if rows is None else int(rows)
    _lib.call("leat_quantize_q8", src.data_ptr(), done, n, _lib.ptr(weight), eps, q.data_ptr(), d.data_ptr(),
              s.data_ptr(), _lib.stream(src.device))  # fmt: skip
    return q, d, s


# ------------------------------------------------------------------------ decode (matvec)


def supports_matvec(x: torch.Tensor, w: QTensor) -> bool:
    """1..MATVEC_TOKENS tokens and rows of whole 64-weight units (leat/kernels/matvec.py:355-359),
    in a type these kernels decode, on a gfx950 GPU."""
    if not (0 < _rows_of(x) <= MATVEC_TOKENS):
        return False
    return w.type in MATVEC_TYPES and w.shape[1] % 64 == 0 and _on_gfx950(x)


def matvecs(
    x: torch.Tensor, *ws: QTensor, norm: Norm | None = None, residual: torch.Tensor | None = None
) -> list[torch.Tensor]:
    """The products x @ w.T of a few tokens with each w (leat/kernels/matvec.py:362-380). x is
    quantized once for all of them, after RMSNorm with `norm` if given. A `residual` is added by
    the kernel and is only allowed with a single matrix. Matrices of one type share one launch."""
    if residual is not None and len(ws) != 1:
        raise ValueError("matvecs adds a residual to the product of one matrix only")
    tokens, cols = _rows_of(x), x.shape[-1]
    device = x.device
    outs = [torch.empty(tokens * w.shape[0], dtype=torch.float32, device=device) for w in ws]
    lead = x.shape[:-1]
    one_type = all(w.type == ws[0].type for w in ws) and len(ws) <= 4
    src = _f32(x)
    weight, eps = _norm_args(norm)
    few_rows = sum(w.shape[0] for w in ws) <= SELF_QUANTIZED_ROWS
    if one_type and few_rows and _self_quantized(ws[0].type, cols, tokens) and _aligned16(src, weight):
        # one launch: each workgroup quantizes x itself (after the norm), then the products
        stream = _lib.stream(device)
        if residual is None:
            n = len(ws)
            _lib.call("leat_matvecs_f32", n, (ctypes.c_int * n)(*(int(w.type) for w in ws)),
                      (ctypes.c_void_p * n)(*(_blocks(w) for w in ws)), (ctypes.c_int * n)(*(w.shape[0] for w in ws)),
                      cols, src.data_ptr(), tokens, _lib.ptr(weight), eps,
                      (ctypes.c_void_p * n)(*(o.data_ptr() for o in outs)), stream)  # fmt: skip
        else:
            w, out = ws[0], outs[0]
            add = _f32(residual).reshape(-1)
            _lib.call("leat_matvec_f32", int(w.type), _blocks(w), w.shape[0], cols, src.data_ptr(), tokens,
                      _lib.ptr(weight), eps, add.data_ptr(), out.data_ptr(), stream)  # fmt: skip
        return [out.view(*lead, w.shape[0]) for out, w in zip(outs, ws, strict=True)]
    xq, xd, xs = quantize_q8(x.reshape(tokens, cols), norm)
    if residual is None:
        n = len(ws)
        _lib.call("leat_matvecs", n, (ctypes.c_int * n)(*(int(w.type) for w in ws)),
                  (ctypes.c_void_p * n)(*(_blocks(w) for w in ws)), (ctypes.c_int * n)(*(w.shape[0] for w in ws)),
                  cols, xq.data_ptr(), xd.data_ptr(), xs.data_ptr(), tokens,
                  (ctypes.c_void_p * n)(*(o.data_ptr() for o in outs)), _lib.stream(device))  # fmt: skip
    else:
        w, out = ws[0], outs[0]
        add = _f32(residual).reshape(-1)
        _lib.call("leat_matvec", int(w.type), _blocks(w), w.shape[0], cols, xq.data_ptr(), xd.data_ptr(),
                  xs.data_ptr(), tokens, add.data_ptr(), out.data_ptr(), _lib.stream(device))  # fmt: skip
    return [out.view(*lead, w.shape[0]) for out, w in zip(outs, ws, strict=True)]


def matvecs_quantized(
    q8: Q8, tokens: int, cols: int, *ws: QTensor, residual: torch.Tensor | None = None
) -> list[torch.Tensor]:
    """matvecs() of activations already quantized as quantize_q8 makes them, (words, d, s) of
    `tokens` rows of `cols` values (attention_q8's output): the same products, bit for bit, as
    matvecs of the f32 rows those came from, without quantizing them again. Returns (tokens,
    rows) f32 for each w."""
    if residual is not None and len(ws) != 1:
        raise ValueError("matvecs adds a residual to the product of one matrix only")
    xq, xd, xs = q8
    if any(w.shape[1] != cols for w in ws):
        raise ValueError(f"matvecs_quantized: rows of {cols} values against matrices of {[w.shape[1] for w in ws]} columns")
    if xq.numel() != tokens * cols // 4 or xd.numel() != tokens * cols // GROUP or xs.numel() != xd.numel():
        raise ValueError(f"matvecs_quantized: q8 buffers not those of {tokens} rows of {cols} values")
    if residual is not None and residual.numel() != tokens * ws[0].shape[0]:
        raise ValueError("matvecs_quantized: the residual is not the product's shape")
    device = xq.device
    outs = [torch.empty(tokens * w.shape[0], dtype=torch.float32, device=device) for w in ws]
    if residual is None:
        n = len(ws)
        _lib.call("leat_matvecs", n, (ctypes.c_int * n)(*(int(w.type) for w in ws)),
                  (ctypes.c_void_p * n)(*(_blocks(w) for w in ws)), (ctypes.c_int * n)(*(w.shape[0] for w in ws)),
                  cols, xq.data_ptr(), xd.data_ptr(), xs.data_ptr(), tokens,
                  (ctypes.c_void_p * n)(*(o.data_ptr() for o in outs)), _lib.stream(device))  # fmt: skip
    else:
        w, out = ws[0], outs[0]
        add = _f32(residual).reshape(-1)
        _lib.call("leat_matvec", int(w.type), _blocks(w), w.shape[0], cols, xq.data_ptr(), xd.data_ptr(),
                  xs.data_ptr(), tokens, add.data_ptr(), out.data_ptr(), _lib.stream(device))  # fmt: skip
    return [out.view(tokens, w.shape[0]) for out, w in zip(outs, ws, strict=True)]


def supports_qkv_rotate(x: torch.Tensor, q: QTensor, k: QTensor, v: QTensor, cache: torch.Tensor, halves: bool,
                        norm: Norm | None = None) -> bool:  # fmt: skip
    """Whether matvecs(x, q, k, v, norm) and rotate() run as one launch (include/leatmi.h
    leat_qkv_rotate_f32): 1..2 tokens of matrices of one type the self-quantizing kernels take,
    adjacent-pair RoPE, an f16 cache of heads of 16k dimensions."""
    dim, kv_heads = cache.shape[-1], cache.shape[2]
    tokens, cols = _rows_of(x), x.shape[-1]
    shapes = (q.shape[0] % dim == 0 and k.shape[0] == kv_heads * dim and v.shape[0] == kv_heads * dim
              and q.shape[1] == cols == k.shape[1] == v.shape[1])  # fmt: skip
    weight = None if norm is None else norm[0]
    return (not halves and cache.dtype == torch.float16 and cache.is_contiguous() and dim % 16 == 0 and shapes
            and q.type == k.type == v.type and _self_quantized(q.type, cols, tokens)
            and (q.shape[0] + k.shape[0] + v.shape[0]) <= SELF_QUANTIZED_ROWS
            and _aligned16(_f32(x), None if weight is None else _f32(weight)) and _on_gfx950(x))  # fmt: skip


def qkv_rotate(
    x: torch.Tensor, q: QTensor, k: QTensor, v: QTensor, norm: Norm | None, cache: torch.Tensor, slots, positions,
    rope: tuple[tuple[torch.Tensor, torch.Tensor], int] | None,
) -> torch.Tensor:  # fmt: skip
    """matvecs(x, q, k, v, norm=norm) then rotate(q, k, v, cache, slots, positions, rope, False) in
    one launch, bit for bit: x (1, T, cols), the f16 cache (2, slots, KV_H, positions, D) filled at
    each token's slot and position. Returns q rotated (1, H, T, D) f32."""
    _lib.require_device(x)
    tokens, cols = _rows_of(x), x.shape[-1]
    _, cache_slots, kv_heads, cache_positions, dim = cache.shape
    heads = q.shape[0] // dim
    device = x.device
    src = _f32(x).contiguous()
    weight, eps = _norm_args(norm)
    out = torch.empty(heads * tokens * dim, dtype=torch.float32, device=device)
    slot_rows = _device_rows(slots, device)
    pos_rows = _device_rows(positions, device)
    if rope is None:
        cos = sin = None
        rotated = 0
    else:
        (cos, sin), rotated = (t.float().contiguous() for t in rope[0]), rope[1]
        if cos.shape[0] < cache_positions:
            raise _lib.LeatError("qkv_rotate: the RoPE tables must cover every position of the cache")
    _lib.call("leat_qkv_rotate_f32", int(q.type), _blocks(q), _blocks(k), _blocks(v), heads, kv_heads, dim, cols,
              src.data_ptr(), tokens, _lib.ptr(weight), eps, _lib.ptr(cos), _lib.ptr(sin), rotated,
              slot_rows.data_ptr(), pos_rows.data_ptr(), out.data_ptr(), cache.data_ptr(), cache_slots,
              cache_positions, _lib.stream(device))  # fmt: skip
    return out.view(1, heads, tokens, dim)


def _device_rows(values, device: torch.device) -> torch.Tensor:
    # an int32 device tensor of per-token slots or positions (a tensor as given, or a list)
    if isinstance(values, torch.Tensor):
        return values.to(device=device, dtype=torch.int32).contiguous()
    return torch.tensor(list(values), dtype=torch.int32, device=device)


def swiglu(
    x: torch.Tensor, gate: QTensor, up: QTensor, norm: Norm | None = None, kind: str = "silu"
) -> torch.Tensor:
    """glu(kind) of the gate and up products of a few tokens, both matrices (same type and shape)
    read by one kernel from one quantization of x, after RMSNorm with `norm` if given
    (leat/kernels/matvec.py:383-395)."""
    return _swiglu(x, gate, up, norm, kind, q8_out=False)[0]


def _swiglu(x, gate, up, norm, kind, q8_out):
    # the GLU's f32 outputs and, when asked, their q8 (quantize_q8 of them) for the down product
    tokens, cols = _rows_of(x), x.shape[-1]
    rows = gate.shape[0]
    device = x.device
    out = torch.empty(tokens * rows, dtype=torch.float32, device=device)
    src = _f32(x)
    weight, eps = _norm_args(norm)
    if _self_quantized(gate.type, cols, tokens) and _aligned16(src, weight):
        q8 = _q8_buffers(tokens, rows, device) if q8_out and rows % 32 == 0 else None
        hq, hd, hs = (None, None, None) if q8 is None else (t.data_ptr() for t in q8)
        _lib.call("leat_glu_matvec_f32", int(gate.type), _blocks(gate), _blocks(up), rows, cols, src.data_ptr(),
                  tokens, _lib.ptr(weight), eps, GLU_KINDS[kind], out.data_ptr(), hq, hd, hs,
                  _lib.stream(device))  # fmt: skip
        return out.view(*x.shape[:-1], rows), q8
    xq, xd, xs = quantize_q8(x.reshape(tokens, cols), norm)
    if q8_out and rows % 32 == 0:
        # the outputs' q8 for the down product from the GLU launch itself where its kernel can
        q8 = _q8_buffers(tokens, rows, device)
        _lib.call("leat_glu_matvec_q8", int(gate.type), _blocks(gate), _blocks(up), rows, cols, xq.data_ptr(),
                  xd.data_ptr(), xs.data_ptr(), tokens, GLU_KINDS[kind], out.data_ptr(), *(t.data_ptr() for t in q8),
                  _lib.stream(device))  # fmt: skip
        return out.view(*x.shape[:-1], rows), q8
    _lib.call("leat_glu_matvec", int(gate.type), _blocks(gate), _blocks(up), rows, cols, xq.data_ptr(),
              xd.data_ptr(), xs.data_ptr(), tokens, GLU_KINDS[kind], out.data_ptr(), _lib.stream(device))  # fmt: skip
    return out.view(*x.shape[:-1], rows), None


def matvec_f32x(x: torch.Tensor, w: QTensor, residual: torch.Tensor | None = None) -> torch.Tensor:
    """x @ w.dequant().T for up to 8 (or 16) tokens whose activations stay f32: the
    LEAT_KERNELS=ref product (leat/ops.py:35-38), one kernel reading each block once."""
    _lib.require_device(x)
    tokens, cols = _rows_of(x), x.shape[-1]
    src = _f32(x)
    out = torch.empty(tokens * w.shape[0], dtype=torch.float32, device=x.device)
    add = None if residual is None else _f32(residual).reshape(-1)
    _lib.call("leat_matvec_f32x", int(w.type), _blocks(w), w.shape[0], cols, src.data_ptr(), tokens,
              _lib.ptr(add), out.data_ptr(), _lib.stream(x.device))  # fmt: skip
    return out.view(*x.shape[:-1], w.shape[0])


def group_dots(xq: torch.Tensor, w: QTensor, tokens: int) -> torch.Tensor:
    """Parity probe: the exact int32 sums the matvec kernels scale, per token, row and scale
    span (32 weights for Q4_K and Q8_0, 16 for Q6_K). Returns (tokens, rows, spans) int32."""
    rows, cols = w.shape
    spans = cols // (16 if w.type == GGMLType.Q6_K else 32)
    out = torch.empty(tokens * rows * spans, dtype=torch.int32, device=xq.device)
    _lib.call("leat_group_dots", int(w.type), _blocks(w), rows, cols, xq.data_ptr(), tokens, out.data_ptr(),
              _lib.stream(xq.device))  # fmt: skip
    return out.view(tokens, rows, spans)


# ---------------------------------------------------------------------- prefill (matmul)


def _single_sequence(x: torch.Tensor) -> bool:
    # (1, T, dim) or (T, dim): every axis before the tokens is 1 (leat/kernels/common.py:60-62)
    return all(size == 1 for size in x.shape[:-2])


def matmul_fits(ggml_type: GGMLType, rows: int, cols: int) -> bool:
    """Shapes the prefill tiles take (leat/kernels/matmul.py:1041-1044): rows in 64s, rows of
    whole 256-weight steps, and row byte lengths that keep every block 4-byte aligned."""
    if ggml_type not in MATVEC_TYPES or rows % 64 != 0:
        return False
    if ggml_type not in KERNEL_TYPES:  # the decode tasks, 8 tokens a launch: whole pairs of blocks
        return cols % 64 == 0 and cols % BLOCK[ggml_type][0] == 0
    if cols % 256 != 0:
        return False
    elements, size = BLOCK[ggml_type]
    return cols // elements * size % 4 == 0


def supports_matmul(x: torch.Tensor, w: QTensor) -> bool:
    """One sequence's tokens and a matrix the tiles fit (leat/kernels/matmul.py:1046-1048), on a
    gfx950 GPU."""
    return _single_sequence(x) and matmul_fits(w.type, *w.shape) and _on_gfx950(x)


def _workspace(ggml_type: GGMLType, rows: int, cols: int, tokens: int, gated: bool, device) -> tuple[int | None, int]:
    # (address, bytes) of the workspace a split prefill product takes (matmul.py:1005-1010), or none
    size = _lib.workspace_bytes(ggml_type, rows, cols, tokens, gated)
    if size == 0:
        return None, 0
    return torch.empty(size, dtype=torch.uint8, device=device).data_ptr(), size


def _matmul(w: QTensor, q8: Q8, tokens: int, residual: torch.Tensor | None) -> torch.Tensor:
    xq, xd, xs = q8
    rows, cols = w.shape
    out = torch.empty(tokens * rows, dtype=torch.float32, device=xq.device)
    add = None if residual is None else _f32(residual).reshape(-1)
    ws, size = _workspace(w.type, rows, cols, tokens, False, xq.device)
    _lib.call("leat_matmul", int(w.type), _blocks(w), rows, cols, xq.data_ptr(), xd.data_ptr(), xs.data_ptr(),
              tokens, _lib.ptr(add), out.data_ptr(), ws, size, _lib.stream(xq.device))  # fmt: skip
    return out


def matmuls(
    x: torch.Tensor, *ws: QTensor, norm: Norm | None = None, residual: torch.Tensor | None = None
) -> list[torch.Tensor]:
    """The products x @ w.T of a prompt's tokens x (1, T, n) with each w on matrix cores
    (leat/kernels/matmul.py:1051-1066). x is quantized once, after RMSNorm with `norm` if given;
    a `residual` is added by the kernel and needs a single matrix."""
    if residual is not None and len(ws) != 1:
        raise ValueError("matmuls adds a residual to the product of one matrix only")
    tokens, cols = _rows_of(x), x.shape[-1]
    q8 = quantize_q8(x.reshape(tokens, cols), norm)
    return [_matmul(w, q8, tokens, residual).view(*x.shape[:-1], w.shape[0]) for w in ws]


def feed_forward(
    x: torch.Tensor, gate: QTensor, up: QTensor, down: QTensor, norm: Norm, kind: str = "silu",
    residual: bool = True,
) -> torch.Tensor:  # fmt: skip
    """A gated MLP: quantize rms_norm(x, *norm); one kernel for the gate and up products and
    their glu(kind); quantize that; the down product, plus x when `residual`. gate and up share a
    type and shape. A prompt's tokens run on matrix cores (leat/kernels/matmul.py:1069-1081). Up
    to MATVEC_TOKENS tokens run on the decode kernels (swiglu, then the down product), the GLU
    writing the down product's q8 input with its outputs."""
    tokens, cols = _rows_of(x), x.shape[-1]
    rows = gate.shape[0]
    add = _f32(x).reshape(-1) if residual else None
    if tokens <= MATVEC_TOKENS:
        hidden, q8 = _swiglu(x, gate, up, norm, kind, q8_out=True)
        if q8 is None:
            q8 = quantize_q8(hidden.reshape(tokens, rows))
        xq, xd, xs = q8
        out = torch.empty(tokens * down.shape[0], dtype=torch.float32, device=x.device)
        _lib.call("leat_matvec", int(down.type), _blocks(down), down.shape[0], rows, xq.data_ptr(), xd.data_ptr(),
                  xs.data_ptr(), tokens, _lib.ptr(add), out.data_ptr(), _lib.stream(x.device))  # fmt: skip
        return out.view(*x.shape[:-1], down.shape[0])
    xq, xd, xs = quantize_q8(x.reshape(tokens, cols), norm)
    ws, size = _workspace(gate.type, rows, cols, tokens, True, x.device)
    if rows % GROUP == 0:  # the GLU writes the down product's q8 input (Q4_K: in its own kernel)
        i32, f32 = dict(dtype=torch.int32, device=x.device), dict(dtype=torch.float32, device=x.device)
        hq8 = (torch.empty(tokens * rows // 4, **i32), torch.empty(tokens * rows // GROUP, **f32),
               torch.empty(tokens * rows // GROUP, **f32))  # fmt: skip
        # the f32 outputs, which Q4_K's prefill kernel can skip past FEW_TOKENS
        keep = gate.type != GGMLType.Q4_K or tokens <= FEW_TOKENS
        hidden = torch.empty(tokens, rows, **f32) if keep else None
        _lib.call("leat_glu_matmul_q8", int(gate.type), _blocks(gate), _blocks(up), rows, cols, xq.data_ptr(),
                  xd.data_ptr(), xs.data_ptr(), tokens, GLU_KINDS[kind], _lib.ptr(hidden), hq8[0].data_ptr(),
                  hq8[1].data_ptr(), hq8[2].data_ptr(), ws, size, _lib.stream(x.device))  # fmt: skip
    else:
        hidden = torch.empty(tokens, rows, dtype=torch.float32, device=x.device)
        _lib.call("leat_glu_matmul", int(gate.type), _blocks(gate), _blocks(up), rows, cols, xq.data_ptr(),
                  xd.data_ptr(), xs.data_ptr(), tokens, GLU_KINDS[kind], hidden.data_ptr(), ws, size,
                  _lib.stream(x.device))  # fmt: skip
        hq8 = quantize_q8(hidden)
    out = _matmul(down, hq8, tokens, x if residual else None)
    return out.view(*x.shape[:-1], down.shape[0])


# ------------------------------------------------------------------------ experts (MoE)


def route(scores: torch.Tensor, used: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Each token's `used` top experts from its row of `scores` (T, experts)
    (leat/kernels/experts.py:163-172). Returns ids (T·used) int32 in descending order of score,
    equal scores taken lowest id first, -inf and NaN ranked as the lowest finite score; and the
    softmax of the chosen scores (T·used) f32."""
    _lib.require_device(scores)
    tokens, experts = scores.shape
    src = _f32(scores)
    ids = torch.empty(tokens * used, dtype=torch.int32, device=src.device)
    weights = torch.empty(tokens * used, dtype=torch.float32, device=src.device)
    _lib.call("leat_route", src.data_ptr(), tokens, experts, used, ids.data_ptr(), weights.data_ptr(),
              _lib.stream(src.device))  # fmt: skip
    return ids, weights


def supports_scores(x: torch.Tensor, router: QTensor) -> bool:
    """An F32 router whose rows are whole 16-byte loads (leat/kernels/experts.py:110-112), on a
    gfx950 GPU."""
    return router.type == GGMLType.F32 and router.shape[1] % 4 == 0 and _on_gfx950(x)


def scores(x: torch.Tensor, norm: Norm, router: QTensor) -> torch.Tensor:
    """The router's scores of the experts for tokens x (1, T, dim): rms_norm(x, *norm) @ router.T
    in f32 (leat/kernels/experts.py:115-124), one kernel: the norm's sum of squares and the
    router rows' dot products with x * weight, scaled by the inverse root mean square."""
    _lib.require_device(x)
    dim = x.shape[-1]
    tokens, experts = _rows_of(x), router.shape[0]
    src = _aligned(_f32(x).reshape(tokens, dim))
    weight = _aligned(_f32(norm[0]))
    table = _aligned(router.data.reshape(experts, dim).float())
    out = torch.empty(tokens, experts, dtype=torch.float32, device=x.device)
    _lib.call("leat_scores", src.data_ptr(), tokens, dim, weight.data_ptr(), float(norm[1]), table.data_ptr(),
              experts, out.data_ptr(), _lib.stream(x.device))  # fmt: skip
    return out.view(*x.shape[:-1], experts)


def _decode_tasks_fit(ggml_type: GGMLType, length: int) -> bool:
    # a row length the decode tasks cover: whole 256-weight blocks, or pairs of Q8_0 blocks
    step = 64 if ggml_type == GGMLType.Q8_0 else 256
    return length > 0 and length % step == 0


def supports_mixture(x: torch.Tensor, gate: QTensor, up: QTensor | None, down: QTensor) -> bool:
    """Expert stacks these kernels take (leat/kernels/experts.py:288-296): gate (and up, alike)
    (experts, rows, cols), down (experts, cols, rows); with up None, gate stacks gate and up rows.
    Types the kernels decode, at most 256 experts, rows of whole decode tasks, tokens of one
    sequence, on a gfx950 GPU."""
    experts, rows, cols = gate.shape
    if up is None:
        rows //= 2
    elif up.type != gate.type or up.shape != gate.shape:
        return False
    if gate.type not in KERNEL_TYPES or down.type not in KERNEL_TYPES or down.shape != (experts, cols, rows):
        return False
    if experts > 256 or not (_decode_tasks_fit(gate.type, cols) and _decode_tasks_fit(down.type, rows)):
        return False
    return _single_sequence(x) and _on_gfx950(x)



def _fused_mixture_fits(ggml_type: int, cols: int, rows: int, experts: int, used: int, tokens: int) -> bool:
    """Whether leat_experts_glu_f32 takes the decode mixture's first steps in one launch
    (include/leatmi.h): 1..8 tokens, hidden rows in 32s, rows of at most 4 turns of a wave's
    64 tasks (8192 weights)."""
    if not (1 <= tokens <= MATVEC_TOKENS and rows % 32 == 0 and experts <= 256 and used <= 64):
        return False
    if ggml_type == GGMLType.Q4_K:
        ok, tasks = cols % 256 == 0, cols // 32
    elif ggml_type == GGMLType.Q6_K:
        ok, tasks = cols % 512 == 0, cols // 32
    elif ggml_type == GGMLType.Q8_0:
        ok, tasks = cols % 64 == 0, cols // 64
    else:
        return False
    return ok and tasks <= 4 * 64


def mixture(
    x: torch.Tensor, scores: torch.Tensor, gate: QTensor, up: QTensor | None, down: QTensor, used: int,
    norm: Norm, kind: str = "silu", scales: torch.Tensor | None = None, residual: bool = True,
    biases: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None, live: int | None = None,
) -> torch.Tensor:  # fmt: skip
    """The mixture-of-experts MLP of tokens x (1, T, dim) (leat/kernels/experts.py:299-377).

    Steps, all on this library's kernels:
    1. route `scores` (1, T, experts);
    2. quantize rms_norm(x, *norm);
    3. every chosen expert's gate+up+glu(kind), reading each expert once for all its tokens,
       with the (gate, up, down) `biases` (experts, rows) if given;
    4. quantize those hidden rows;
    5. the experts' down products, summed per token with the routing weights (times `scales[e]`
       if given), plus x when `residual`.
    For decode (up to 8 tokens, shapes _fused_mixture_fits takes) steps 1-4 are one launch.

    With up None, gate stacks each expert's gate rows, then its up rows. Tokens past the first
    `live` are batch padding: no expert runs for them and their mixture is 0."""
    _, tokens, dim = x.shape
    if not 0 < used <= MAX_USED:
        raise _lib.LeatError(f"mixture: {used} experts a token (the kernels take 1..{MAX_USED})")
    real = tokens if live is None else int(live)
    chunk = MAX_PAIRS // used
    if real > chunk:  # a long prompt: the expert launches take at most MAX_PAIRS pairs each
        out = torch.cat([
            mixture(x[:, at : min(at + chunk, real)], scores.reshape(1, tokens, -1)[:, at : min(at + chunk, real)], gate,
                    up, down, used, norm, kind, scales, residual, biases)
            for at in range(0, real, chunk)
        ] + ([x[:, real:].float() if residual else torch.zeros_like(x[:, real:], dtype=torch.float32)]
             if real < tokens else []), dim=1)  # fmt: skip
        return out
    device = x.device
    rows = down.shape[2]
    flat_x = _f32(x.reshape(tokens, dim))
    out = flat_x.clone() if residual else torch.zeros_like(flat_x)
    if real == 0:
        return out.view(x.shape)
    pairs = real * used
    experts = gate.shape[0]
    gate_b, up_b, down_b = (None, None, None) if biases is None else (_f32(b).reshape(-1) for b in biases)
    stream = _lib.stream(device)
    route_scores = _f32(scores.reshape(tokens, -1)[:real])
    norm_w, eps = _norm_args(norm)
    aligned = flat_x.data_ptr() % 16 == 0 and (norm_w is None or norm_w.data_ptr() % 16 == 0)
    if _fused_mixture_fits(gate.type, dim, rows, experts, used, real) and aligned:
        # decode: routing, norm + quantize, the experts' gate+up+GLU and the quantized hidden rows
        # in one launch
        ids = torch.empty(pairs, dtype=torch.int32, device=device)
        weights = torch.empty(pairs, dtype=torch.float32, device=device)
        hq, hd, hs = _q8_buffers(pairs, rows, device)
        _lib.call("leat_experts_glu_f32", int(gate.type), _blocks(gate), None if up is None else _blocks(up), experts,
                  rows, dim, flat_x.data_ptr(), real, _lib.ptr(norm_w), eps, route_scores.data_ptr(), used,
                  _lib.ptr(gate_b), _lib.ptr(up_b), GLU_KINDS[kind], ids.data_ptr(), weights.data_ptr(), None,
                  hq.data_ptr(), hd.data_ptr(), hs.data_ptr(), stream)  # fmt: skip
    else:
        ids, weights = route(route_scores, used)
        xq, xd, xs = quantize_q8(flat_x[:real], norm)
        hidden = torch.empty(pairs * rows, dtype=torch.float32, device=device)
        _lib.call("leat_experts_glu", int(gate.type), _blocks(gate), None if up is None else _blocks(up), experts,
                  rows, dim, xq.data_ptr(), xd.data_ptr(), xs.data_ptr(), ids.data_ptr(), pairs, used,
                  _lib.ptr(gate_b), _lib.ptr(up_b), GLU_KINDS[kind], hidden.data_ptr(), stream)  # fmt: skip
        hq, hd, hs = quantize_q8(hidden.view(pairs, rows))
    expert_scale = None if scales is None else _f32(scales)
    _lib.call("leat_experts_down", int(down.type), _blocks(down), experts, dim, rows, hq.data_ptr(),
              hd.data_ptr(), hs.data_ptr(), ids.data_ptr(), weights.data_ptr(), real, used, _lib.ptr(expert_scale),
              _lib.ptr(down_b), _lib.ptr(flat_x if residual else None), out.data_ptr(), stream)  # fmt: skip
    return out.view(x.shape)


__all__ = [
    "argmax", "attention", "attention_q8", "attention_workspace", "embedding", "rotate", "supports_argmax", "supports_attention", "supports_embedding",
    "supports_rotate",
    "FEW_TOKENS", "GROUP", "MATVEC_TOKENS", "MAX_PAIRS", "MAX_USED", "SELF_QUANTIZED_ROWS", "SELF_QUANTIZED_TOKENS", "feed_forward", "group_dots", "matmul_fits", "matmuls", "qkv_rotate", "supports_qkv_rotate",
    "matvec_f32x", "matvecs", "matvecs_quantized", "mixture", "quantize_q8", "route", "scores", "supports_matmul", "supports_matvec",
    "supports_mixture", "supports_scores", "swiglu",
]  # fmt: skip
