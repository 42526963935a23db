"""The decode step's attention and its inputs (leat/kernels/attention.py:226-279, 656-782), the
greedy choice of the next token (leat/kernels/argmax.py:14-59) and the embedding gather
(leat/ops.py:166-178), on the HIP kernels of libleatmi.so.

Rows carry one query token each, as leat's FlashDecoding path takes them: row t attends over
positions 0..positions[t] of cache slot slots[t]. Slots and positions may be device tensors, so a
captured graph replays with whatever positions the tensors hold.
"""

from __future__ import annotations

import torch

from leat_amd import _lib
from leat_amd.quant import BLOCK, DEQUANT_TYPES, NATIVE, QTensor

HEAD_DIM = 128  # the head dimension the attention kernel takes


def _on_gfx950(x: torch.Tensor) -> bool:
    if not x.is_cuda:
        return False
    index = torch.cuda.current_device() if x.device.index is None else x.device.index
    return _lib.device_ok(index)


def _rows_tensor(values, device: torch.device) -> torch.Tensor:
    # an int32 device tensor of per-row slots or positions (a tensor as given, or a list)
    if isinstance(values, torch.Tensor):
        return values.to(device=device, dtype=torch.int32).contiguous()
    return torch.tensor(list(values), dtype=torch.int32, device=device)


def supports_rotate(q: torch.Tensor, cache: torch.Tensor) -> bool:
    """An f16 cache of whole pairs of dimensions, on a gfx950 GPU (leat/kernels/attention.py:760-765)."""
    return cache.dtype == torch.float16 and cache.shape[-1] % 2 == 0 and _on_gfx950(q)


def rotate(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cache: torch.Tensor, slots, positions,
    rope: tuple[tuple[torch.Tensor, torch.Tensor], int] | None, halves: bool,
) -> tuple[torch.Tensor, torch.Tensor]:  # fmt: skip
    """q (1, T, H, D), k and v (1, T, KV_H, D): the first R dimensions of q and k turned by RoPE's
    tables (positions, R/2) for rope ((cos, sin), R), pairs of adjacent dimensions or with
    `halves` dimensions i and i + R/2; k and v stored in the f16 cache (2, slots, KV_H, positions,
    D) at each token's slot and position. Returns q rotated (1, H, T, D) f32, and the cache."""
    _lib.require_device(q)
    _, tokens, heads, dim = q.shape
    kv_heads = k.shape[2]
    _, cache_slots, cache_kv, cache_positions, cache_dim = cache.shape
    if cache_kv != kv_heads or cache_dim != dim or not cache.is_contiguous():
        raise _lib.LeatError("rotate: the cache does not match the keys' heads and dimensions")
    device = q.device
    srcs = [t.reshape(-1).float().contiguous() for t in (q, k, v)]
    out = torch.empty(heads * tokens * dim, dtype=torch.float32, device=device)
    slot_rows, pos_rows = _rows_tensor(slots, device), _rows_tensor(positions, device)
    if rope is None:
        cos = sin = None
        rotated = 0
    else:
        (cos, sin), rotated = (t.float().contiguous() for t in rope[0]), rope[1]
        if cos.shape[0] < cache_positions:
            raise _lib.LeatError("rotate: the RoPE tables must cover every position of the cache")
    _lib.call("leat_rotate", *(t.data_ptr() for t in srcs), tokens, heads, kv_heads, dim, _lib.ptr(cos), _lib.ptr(sin),
              rotated, int(halves), slot_rows.data_ptr(), pos_rows.data_ptr(), out.data_ptr(), cache.data_ptr(),
              cache_slots, cache_positions, _lib.stream(device))  # fmt: skip
    return out.view(1, heads, tokens, dim), cache


def supports_attention(q: torch.Tensor, cache: torch.Tensor) -> bool:
    """One query token a row over an f16 cache of 128-dimension heads, 1, 2, 4 or 8 query heads a
    kv head (leat/kernels/attention.py:214-223), on a gfx950 GPU."""
    heads, dim = q.shape[1], q.shape[-1]
    kv_heads = cache.shape[2]
    group = heads // kv_heads if heads % kv_heads == 0 else 0
    return (cache.dtype == torch.float16 and dim == HEAD_DIM and cache.shape[-1] == HEAD_DIM and group in (1, 2, 4, 8)
            and q.shape[0] == 1 and _on_gfx950(q))  # fmt: skip


def attention_workspace(rows: int, heads: int, max_length: int, device) -> torch.Tensor:
    """A workspace for attention() calls of up to `rows` rows of `heads` query heads and rows of at
    most `max_length` keys, reusable by such calls one after another on a stream. Calls that may
    overlap need workspaces of their own."""
    size = int(_lib.lib().leat_attention_workspace(rows, heads, max_length))
    return torch.empty(max(size, 4), dtype=torch.uint8, device=device)


def attention(
    q: torch.Tensor, cache: torch.Tensor, slots, lengths, scale: float, max_length: int | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:  # fmt: skip
    """FlashDecoding (leat/kernels/attention.py:226-279): q (1, H, T, D), a query token a row; row t
    over the first lengths[t] positions of slot slots[t] of the cache (2, slots, KV_H, positions,
    D), scores q.k * scale. `max_length` bounds every length (the cache's positions if not
    given) and sizes the launch. `workspace` is one from attention_workspace() for at least these
    rows, heads and max_length (a new one is made if not given). Returns (1, T, H * D) f32."""
    out, _ = _attention(q, cache, slots, lengths, scale, max_length, workspace, False)
    return out


def attention_q8(
    q: torch.Tensor, cache: torch.Tensor, slots, lengths, scale: float, max_length: int | None = None,
    workspace: torch.Tensor | None = None,
) -> tuple[torch.Tensor, tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:  # fmt: skip
    """attention(), and the q8 of its output as quantize_q8 would make it of the (T, H * D) rows,
    written by the attention kernels themselves (include/leatmi.h leat_attention_q8): for the
    q8-input product that follows."""
    return _attention(q, cache, slots, lengths, scale, max_length, workspace, True)


def _attention(q, cache, slots, lengths, scale, max_length, workspace, q8: bool):
    _lib.require_device(q)
    _, heads, rows, dim = q.shape
    _, cache_slots, kv_heads, cache_positions, _ = cache.shape
    device = q.device
    longest = cache_positions if max_length is None else int(max_length)
    size = int(_lib.lib().leat_attention_workspace(rows, heads, longest))
    if workspace is None:
        work = torch.empty(max(size, 4), dtype=torch.uint8, device=device)
    else:
        work = workspace
        if work.dtype != torch.uint8 or not work.is_contiguous() or work.numel() < size or work.device != device:
            raise _lib.LeatError("attention: the workspace is not one of attention_workspace() for these rows")
        size = work.numel() // 4 * 4
    n = rows * heads * dim
    out = torch.empty(n, dtype=torch.float32, device=device)
    src = q.float().contiguous()
    slot_rows, length_rows = _rows_tensor(slots, device), _rows_tensor(lengths, device)
    args = (src.data_ptr(), cache.data_ptr(), cache_slots, kv_heads, cache_positions, dim, rows, heads,
            slot_rows.data_ptr(), length_rows.data_ptr(), longest, float(scale), work.data_ptr(), size, out.data_ptr())  # fmt: skip
    packed = None
    if q8:
        packed = (torch.empty(n // 4, dtype=torch.int32, device=device), torch.empty(n // 32, dtype=torch.float32, device=device),
                  torch.empty(n // 32, dtype=torch.float32, device=device))  # fmt: skip
        _lib.call("leat_attention_q8", *args, *(t.data_ptr() for t in packed), _lib.stream(device))
    else:
        _lib.call("leat_attention", *args, _lib.stream(device))
    return out.view(1, rows, heads * dim), packed


def supports_argmax(x: torch.Tensor) -> bool:
    """Rows of values on a gfx950 GPU (leat/kernels/argmax.py:48-50)."""
    return x.ndim == 2 and _on_gfx950(x)


def argmax(x: torch.Tensor) -> torch.Tensor:
    """The index of the largest value of each row of x (B, V), the first one among equal values,
    NaN never chosen: (B, 1) int32 (leat/kernels/argmax.py:53-59)."""
    _lib.require_device(x)
    rows, n = x.shape
    src = x.float().contiguous()
    size = int(_lib.lib().leat_argmax_workspace(rows))
    work = torch.empty(max(size, 8), dtype=torch.uint8, device=x.device)
    out = torch.empty(rows, dtype=torch.int32, device=x.device)
    _lib.call("leat_argmax", src.data_ptr(), rows, n, work.data_ptr(), size, out.data_ptr(), _lib.stream(x.device))
    return out.view(rows, 1)


def supports_embedding(w: QTensor) -> bool:
    """A matrix in a type these kernels decode (rows whole numbers of blocks)."""
    return w.type in DEQUANT_TYPES and w.shape[1] % BLOCK[w.type][0] == 0 and _on_gfx950(w.data)


def embedding(tokens: torch.Tensor, w: QTensor) -> torch.Tensor:
    """The rows of w (vocab, dim) of token ids (…), decoded to f32: (…, dim) (leat/ops.py:166-178)."""
    ids = tokens.to(device=w.data.device, dtype=torch.int32).contiguous()
    vocab, dim = w.shape
    if w.type in NATIVE:
        return w.data.reshape(vocab, dim)[ids.long()].float()
    out = torch.empty(ids.numel() * dim, dtype=torch.float32, device=w.data.device)
    _lib.call("leat_embedding", int(w.type), w.data.data_ptr(), vocab, dim, ids.data_ptr(), ids.numel(), out.data_ptr(),
              _lib.stream(w.data.device))  # fmt: skip
    return out.view(*tokens.shape, dim)
