"""Benchmark: weight-stream GB/s (% of HBM peak) and decode tok/s of the quantized-weight path,
Llama-3-8B Q4_K_M shapes.

Headline (config 2, B = 1): a step is one decode token's pass over the linear layers of all 32
layers of a random-init Llama-3-8B-shaped model in Q4_K_M: per layer norm+quantize, q/k/v in one
launch, quantize, o (+residual), norm+quantize, gate+up+SiLU-GLU in one launch, quantize, down
(+residual), exactly as leat's decode step calls them (leat/model.py:497-558 via
leat/ops.py:23-55), the attention output standing in with q's product. Weights are 32 distinct
layers of seeded synthetic blocks (4.41 GB, far beyond the 256 MB MALL), resident in HBM before
the timed region; each step is one HIP-graph replay. `value` is weight bytes per step / step time,
as leat's bench counts weight GB/s (leat/bench.py:71-82); `linear_tok_s` is that step's rate (the
linear layers only). The same step runs at B = 4, 8 and 16 ("b4", "b8", "b16"). The roofline
object is for the dominant kernel (gate+up GLU): a step's 32 launches of it back to back in a HIP
graph, timed with HIP events on their stream.

Beside it, as sub-objects: "decode" (config 3: the full single-stream decode step of the model,
embedding to argmax with attention over the f16 KV cache and the Q6_K output head, at 1 and 4095
cached positions: true decode tok/s), "prefill" (config 4: 512 tokens through a layer's FFN on
matrix cores, TOPS against the int8 MFMA peak; and the down product at 8, 16 and 64 tokens, the
few-token and split schedules), "moe" (config 5: a Qwen3-30B-A3B-style mixture at B = 1 and 8),
and "cpu_baseline": the C restatement of leat's LEAT_KERNELS=ref product (oracle/leat_ref.c) on
config 1 (Q8_0 4096 x 4096) and on one config-2 layer, with all the host's threads and with one.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--seed S] [--no-cpu]
                    [--legs decode,prefill,moe,batches] [--copy-probe]
"""

from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HIDDEN, FFN, KV, LAYERS = 4096, 14336, 1024, 32
Q4_K, Q6_K = 12, 14
HBM_PEAK_GBS = 8000.0
METRIC = "weight-stream GB/s (% HBM peak) + decode tok/s, Llama-3-8B Q4_K_M shape, B=1/8"
# (name, type, rows, cols) of a layer's matrices (config 2 of the benchmark)
MATRICES = [
    ("q", Q4_K, HIDDEN, HIDDEN), ("k", Q4_K, KV, HIDDEN), ("v", Q4_K, KV, HIDDEN),
    ("o", Q4_K, HIDDEN, HIDDEN), ("gate", Q4_K, FFN, HIDDEN), ("up", Q4_K, FFN, HIDDEN),
    ("down", Q6_K, HIDDEN, FFN),
]  # fmt: skip
BLOCK = {Q4_K: (256, 144), Q6_K: (256, 210)}


def nbytes(t, rows, cols):
    el, by = BLOCK[t]
    return rows * cols // el * by


LAYER_BYTES = sum(nbytes(t, r, c) for _, t, r, c in MATRICES)  # 137,822,208


def synthetic_weights(torch, t, rows, cols, gen, device):
    # uniform bytes; Q4_K d = f16(|N|*0.002), dmin = f16(|N|*0.001); Q6_K d = f16(|N|*0.002)
    el, by = BLOCK[t]
    n = rows * cols // el
    blocks = torch.randint(0, 256, (n, by), dtype=torch.uint8, device=device, generator=gen)
    def f16_field(scale):
        v = (torch.randn(n, device=device, generator=gen).abs() * scale).half()
        return v.view(torch.uint8).view(n, 2)
    if t == Q4_K:
        blocks[:, 0:2] = f16_field(0.002)
        blocks[:, 2:4] = f16_field(0.001)
    else:
        blocks[:, 208:210] = f16_field(0.002)
    return blocks


class Step:
    """Static buffers and the launch sequence of one decode step at B tokens."""

    def __init__(self, torch, lib, layers, tokens, device):
        self.torch, self.lib, self.layers, self.B = torch, lib, layers, tokens
        f32 = dict(dtype=torch.float32, device=device)
        i32 = dict(dtype=torch.int32, device=device)
        B = tokens
        gen = torch.Generator(device=device).manual_seed(1)
        self.x = [torch.randn(B, HIDDEN, generator=gen, **f32) for _ in range(2)]
        self.norm_w = torch.rand(HIDDEN, generator=gen, **f32) + 0.5
        self.q8 = {n: (torch.empty(B * n // 4, **i32), torch.empty(B * n // 32, **f32), torch.empty(B * n // 32, **f32))
                   for n in (HIDDEN, FFN)}  # fmt: skip
        self.q8b = tuple(torch.empty_like(t) for t in self.q8[HIDDEN])
        self.qkv = [torch.empty(B * r, **f32) for _, _, r, _ in MATRICES[:3]]
        self.h = torch.empty(B, HIDDEN, **f32)
        self.g = torch.empty(B, FFN, **f32)
        # one or two tokens: the kernels quantize their own input, and the GLU its output
        self.self_quantized = tokens <= 2

    def quantize(self, x, n, out, norm):
        q, d, s = out
        w, eps = (self.norm_w.data_ptr(), 1e-5) if norm else (None, 0.0)
        _call(self.lib, "leat_quantize_q8", x.data_ptr(), self.B, n, w, eps, q.data_ptr(), d.data_ptr(),
              s.data_ptr(), self._stream())  # fmt: skip

    def _stream(self):
        return self.torch.cuda.current_stream().cuda_stream

    def glu(self, w):
        # the layer's gate+up GLU launch, as run() issues it
        B, st = self.B, self._stream()
        gq, gd, gs = self.q8[FFN]
        if self.self_quantized:
            _call(self.lib, "leat_glu_matvec_f32", Q4_K, w["gate"].data_ptr(), w["up"].data_ptr(), FFN, HIDDEN,
                  self.h.data_ptr(), B, self.norm_w.data_ptr(), 1e-5, 0, None, gq.data_ptr(), gd.data_ptr(),
                  gs.data_ptr(), st)  # fmt: skip
        else:
            # q8 input; the f32 outputs and their q8 (the down product's input) from the same kernel
            xq, xd, xs = self.q8[HIDDEN]
            _call(self.lib, "leat_glu_matvec_q8", Q4_K, w["gate"].data_ptr(), w["up"].data_ptr(), FFN, HIDDEN,
                  xq.data_ptr(), xd.data_ptr(), xs.data_ptr(), B, 0, self.g.data_ptr(), gq.data_ptr(), gd.data_ptr(),
                  gs.data_ptr(), st)  # fmt: skip

    def run_glu_only(self):
        for w in self.layers:
            self.glu(w)

    def run(self):
        lib, B = self.lib, self.B
        st = self._stream()
        types = (ctypes.c_int * 3)(Q4_K, Q4_K, Q4_K)
        rows = (ctypes.c_int * 3)(HIDDEN, KV, KV)
        outs = (ctypes.c_void_p * 3)(*[o.data_ptr() for o in self.qkv])
        xq, xd, xs = self.q8[HIDDEN]
        aq, ad, as_ = self.q8b
        gq, gd, gs = self.q8[FFN]
        for i, w in enumerate(self.layers):
            x, x_next = self.x[i % 2], self.x[(i + 1) % 2]
            ptrs = (ctypes.c_void_p * 3)(*[w[n].data_ptr() for n in ("q", "k", "v")])
            # norm + quantize + q, k, v; the attention output stands in with q's product (same
            # shape, realistic values); quantize + o + residual; norm + quantize + gate, up, GLU;
            # quantize + down + residual
            if self.self_quantized:
                _call(lib, "leat_matvecs_f32", 3, types, ptrs, rows, HIDDEN, x.data_ptr(), B,
                      self.norm_w.data_ptr(), 1e-5, outs, st)  # fmt: skip
                _call(lib, "leat_matvec_f32", Q4_K, w["o"].data_ptr(), HIDDEN, HIDDEN, self.qkv[0].data_ptr(), B,
                      None, 0.0, x.data_ptr(), self.h.data_ptr(), st)  # fmt: skip
                self.glu(w)
            else:
                self.quantize(x, HIDDEN, self.q8[HIDDEN], True)
                _call(lib, "leat_matvecs", 3, types, ptrs, rows, HIDDEN, xq.data_ptr(), xd.data_ptr(), xs.data_ptr(),
                      B, outs, st)  # fmt: skip
                self.quantize(self.qkv[0], HIDDEN, self.q8b, False)
                _call(lib, "leat_matvec", Q4_K, w["o"].data_ptr(), HIDDEN, HIDDEN, aq.data_ptr(), ad.data_ptr(),
                      as_.data_ptr(), B, x.data_ptr(), self.h.data_ptr(), st)  # fmt: skip
                self.quantize(self.h, HIDDEN, self.q8[HIDDEN], True)
                self.glu(w)
            _call(lib, "leat_matvec", Q6_K, w["down"].data_ptr(), HIDDEN, FFN, gq.data_ptr(), gd.data_ptr(),
                  gs.data_ptr(), B, self.h.data_ptr(), x_next.data_ptr(), st)  # fmt: skip


def _call(lib, name, *args):
    if getattr(lib, name)(*args) != 0:
        raise RuntimeError(f"{name}: {lib.leat_last_error().decode()}")


def glu_bytes(B):
    # algorithmic bytes of one gate+up GLU launch: both matrices, then for one or two tokens the
    # f32 input read (and quantized in the kernel) and the q8 output written (int8 + d + s); for
    # more tokens q8 input, and f32 and q8 outputs
    weights = 2 * nbytes(Q4_K, FFN, HIDDEN)
    if B <= 2:
        return weights + B * HIDDEN * 4 + B * (FFN + FFN // 32 * 8)
    return weights + B * (HIDDEN + HIDDEN // 32 * 8) + B * FFN * 4 + B * (FFN + FFN // 32 * 8)


def measure(torch, lib, layers, B, steps, warmup, device):
    step = Step(torch, lib, layers, B, device)
    step.run()  # eager once: checks every launch
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step.run()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    # the dominant kernel alone: its 32 launches of a step (one per layer, distinct weights)
    # back to back in a graph, timed by events on the stream they run on
    glu_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(glu_graph):
        step.run_glu_only()
    glu_graph.replay()
    torch.cuda.synchronize()
    reps = max(3, steps // 5)
    start.record()
    for _ in range(reps):
        glu_graph.replay()
    end.record()
    torch.cuda.synchronize()
    glu_us = 1000 * start.elapsed_time(end) / (reps * LAYERS)
    weight_bytes = LAYERS * LAYER_BYTES
    gbs = weight_bytes / (ms * 1e-3) / 1e9
    achieved = glu_bytes(B) / (glu_us * 1e-6) / 1e9
    traffic, note = profiled_traffic(f"decode_glu_b{B}")
    return {
        "ms_per_step": ms,
        "weight_gbs": gbs,
        "hbm_frac": gbs / HBM_PEAK_GBS,
        "linear_tok_s": B * 1000.0 / ms,
        "glu_us": glu_us,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": note,
                     "kernel": f"gate+up GLU {'matvec' if B <= 8 else 'matrix-core 16-token tiles'}, Q4_K 2x14336x4096, "
                               f"B={B}" + (" (quantizes its f32 input and its output)" if B <= 2 else ""),
                     "bytes_per_launch": glu_bytes(B)},  # fmt: skip
    }


TRAFFIC_PROFILE = ROOT / "profiles" / "decode_moe_hbm_bytes.md"
# the sources of the decode kernels whose HBM bytes that profile records
TRAFFIC_SOURCES = ["blocks.h", "common.h", "q8.h", "rows.h", "rows.hip", "rowtask.h", "tiles.h", "tiles.hip",
                   "mmv.h", "mmv.hip", "matvec.hip", "experts.hip", "attention.hip"]  # fmt: skip


# the prefill kernels' sources, whose counters profiles/prefill_counters.md records
COUNTER_PROFILE = ROOT / "profiles" / "prefill_counters.md"
COUNTER_SOURCES = ["blocks.h", "common.h", "formats.h", "lds.h", "prefill.h", "prefill.hip", "prefill6.hip", "q8.h",
                   "tasks.h"]  # fmt: skip


def sources_sha(names=None) -> str:
    """A digest of kernel sources (the decode kernels' by default), which a profile records beside
    its figures."""
    digest = hashlib.sha256()
    for name in TRAFFIC_SOURCES if names is None else names:
        digest.update((ROOT / "leat_amd" / "csrc" / name).read_bytes())
    return digest.hexdigest()[:16]


def profiled_counters(kernel: str) -> dict | None:
    """MFMA and VALU busy fractions of `kernel` as the committed rocprofv3 --pmc summary records
    them ("counters <kernel> mfma_util=.. valu_busy=.. coexec=.."), with their source; None when
    it has no line for the kernel or was measured on other kernel sources."""
    try:
        text = COUNTER_PROFILE.read_text()
    except OSError:
        return None
    sha = sources_sha(COUNTER_SOURCES)
    m = re.search(r"^sources sha ([0-9a-f]+)$", text, re.M)
    if not m or m.group(1) != sha:
        return None
    m = re.search(r"^counters " + re.escape(kernel) + r" (.*)$", text, re.M)
    if not m:
        return None
    fields = dict(item.split("=") for item in m.group(1).split())
    return {**{k: float(v) for k, v in fields.items()}, "source": f"profiles/{COUNTER_PROFILE.name}, sources sha {sha}"}


def profiled_traffic(label: str) -> tuple[int | None, str]:
    """HBM bytes per dispatch of a roofline kernel (`label`: decode_glu_b1, moe_glu_b8,
    attention_p4096, ...) as the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary records them
    ("traffic <label> <bytes>", calibrated against a copy of known size), and where that figure
    comes from; None where the summary has no line for it, or was measured on other kernel
    sources than these."""
    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return None, "no traffic profile"
    m = re.search(r"^sources sha ([0-9a-f]+)$", text, re.M)
    if not m or m.group(1) != sources_sha():
        return None, f"{TRAFFIC_PROFILE.name} was measured on other kernel sources (sha {m.group(1) if m else '?'})"
    m = re.search(r"^traffic " + re.escape(label) + r" (\d+)$", text, re.M)
    if not m:
        return None, f"{TRAFFIC_PROFILE.name} has no line for this kernel"
    return int(m.group(1)), f"profiles/{TRAFFIC_PROFILE.name}: rocprofv3 FETCH_SIZE + WRITE_SIZE, sources sha {sources_sha()}"


def _graph_us(torch, fn, reps, inner=1):
    # fn's launches captured once in a HIP graph, replayed `reps` times back to back and timed by
    # events on the stream they run on: microseconds per call of fn, `inner` calls per capture
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(inner):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return 1000 * start.elapsed_time(end) / (reps * inner)


def decode_model(torch, layers, seed, device):
    """Config 3's model around the config-2 layers' weights (shared, not copied): a Q4_K token
    embedding (128256 x 4096), the 32 layers, the final norm and a Q6_K output head (128256 x
    4096), norm weights uniform in [0.5, 1.5), an f16 KV cache of 4096 positions."""
    from leat_amd.model import LLAMA3_8B, Layer, Model, Weights, _synthetic_blocks
    from leat_amd.quant import GGMLType, QTensor

    c = LLAMA3_8B
    gen = torch.Generator(device=device).manual_seed(seed + 7)

    def norm():
        return torch.rand(c.dim, generator=gen, device=device) + 0.5

    def q(w, name):
        t, r, cols = next((t, r, cc) for n, t, r, cc in MATRICES if n == name)
        return QTensor(w[name], GGMLType(t), (r, cols))

    built = [Layer(norm(), q(w, "q"), q(w, "k"), q(w, "v"), q(w, "o"), norm(), q(w, "gate"), q(w, "up"), q(w, "down"))
             for w in layers]  # fmt: skip
    weights = Weights(_synthetic_blocks(GGMLType.Q4_K, c.vocab, c.dim, gen, device), built, norm(),
                      _synthetic_blocks(GGMLType.Q6_K, c.vocab, c.dim, gen, device))  # fmt: skip
    model = Model(c, weights)
    for cache in model.cache:  # cached keys and values of a prompt: N(0, 1) in f16
        cache.normal_(generator=gen)
    return model


def measure_decode(torch, model, steps, device, positions=(1, 4096)):
    """Config 3: the full single-stream decode step (embedding, 32 layers with RoPE + KV store and
    FlashDecoding over the cache, final norm + Q6_K head, argmax) as one HIP-graph replay, at each
    of `positions` cached positions (by default 1 and 4096: the step's token at position 0, then
    at 4095 of a 4096-position cache), each replaying the graph whose length bucket covers it, as
    the engine does (GraphStep: 128 keys, which need no FlashDecoding combine, or the whole
    context). tok/s is one token per step; GB/s counts the matrices
    streamed (layers and head, as leat's bench does) and, for hbm_frac, the keys and values read
    too. FlashDecoding alone over the 32 layers' caches gets a roofline line of its own."""
    from leat_amd.model import GraphStep, weight_bytes

    c = model.config
    step = GraphStep(model, 1, advance=False)  # each replay decodes at the positions the buffer holds
    w_bytes = weight_bytes(model.weights)
    out = {"workload": "llama3.1-8b q4_k_m random-init decode step, B=1 (embedding .. argmax)",
           "weight_bytes_per_token": w_bytes}  # fmt: skip
    for pos in (p - 1 for p in positions):
        step.positions.fill_(pos)
        step.tokens.fill_(128000)
        torch.cuda.synchronize()
        for _ in range(3):
            step.replay(max_length=pos + 1)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            step.replay(max_length=pos + 1)
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        kv = (pos + 1) * c.layers * 2 * c.kv_heads * c.head_dim * 2
        out[f"p{pos + 1}"] = {"positions": pos + 1, "ms_per_token": round(ms, 4), "tok_s": round(1000.0 / ms, 1),
                              "weight_gbs": round(w_bytes / (ms * 1e-3) / 1e9, 1), "kv_bytes": kv,
                              "hbm_frac": round((w_bytes + kv) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}  # fmt: skip
    # FlashDecoding alone (partial sums and their combine) over every layer's cache at the last
    # positions: the keys and values of (pos + 1) positions a layer, read once
    from leat_amd import kernels, ops

    pos = positions[-1] - 1
    q = torch.randn(1, c.heads, 1, c.head_dim, device=device)
    slots = torch.zeros(1, dtype=torch.int32, device=device)
    lengths = torch.full((1,), pos + 1, dtype=torch.int32, device=device)
    work = kernels.attention_workspace(1, c.heads, c.context, device)
    att_us = _graph_us(torch, lambda: [ops.attention(q, cache, None, c.head_dim**-0.5, slots, lengths, c.context, work)
                                       for cache in model.cache], steps) / c.layers  # fmt: skip
    att_bytes = (pos + 1) * 2 * c.kv_heads * c.head_dim * 2 + c.heads * c.head_dim * 4 * 2
    att_gbs = att_bytes / (att_us * 1e-6) / 1e9
    att_traffic, att_note = profiled_traffic(f"attention_p{pos + 1}")
    out["attention"] = {"kernel": f"FlashDecoding over {pos + 1} positions, 32 heads over 8 kv heads of 128 (partial + combine)",
                        "us": round(att_us, 2), "bytes_per_launch": att_bytes,
                        "roofline": {"bound": "hbm", "achieved": att_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                     "frac": att_gbs / HBM_PEAK_GBS, "traffic": att_traffic, "traffic_source": att_note}}  # fmt: skip
    # the largest single product of a step: the Q6_K head (RMSNorm + quantize once, then the
    # product: kernels.matvecs' path for launches of more than SELF_QUANTIZED_ROWS rows)
    x = torch.randn(1, 1, c.dim, device=device)
    norm = (model.weights.output_norm, c.norm_eps)
    head_us = _graph_us(torch, lambda: kernels.matvecs(x, model.weights.output, norm=norm), steps)
    head_bytes = model.weights.output.nbytes + c.dim * 4 + c.vocab * 4
    out["head"] = {"kernel": "Q6_K output head 128256x4096: RMSNorm + quantize_q8, then the q8-input matvec", "us": round(head_us, 2),
                   "gbs": round(head_bytes / (head_us * 1e-6) / 1e9, 1),
                   "frac": round(head_bytes / (head_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}  # fmt: skip
    return out


def measure_few_tokens(torch, lib, w, reps, device):
    """The down product (Q6_K 4096 x 14336, + residual) at 8 tokens (the decode kernels), 16 (the
    16-token matrix-core tiles, leat's FEW_TOKENS) and 64 (prefill tiles, each tile's K steps split
    over workgroups): the few-token and split schedules of leat/kernels/matmul.py:904-964."""
    f32 = dict(dtype=torch.float32, device=device)
    i32 = dict(dtype=torch.int32, device=device)
    gen = torch.Generator(device=device).manual_seed(9)
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    out = {}
    for T in (8, 16, 64):
        h = torch.randn(T, FFN, generator=gen, **f32)
        q, d, sc = torch.empty(T * FFN // 4, **i32), torch.empty(T * FFN // 32, **f32), torch.empty(T * FFN // 32, **f32)
        _call(lib, "leat_quantize_q8", h.data_ptr(), T, FFN, None, 0.0, q.data_ptr(), d.data_ptr(), sc.data_ptr(), st())
        res, y = torch.randn(T, HIDDEN, generator=gen, **f32), torch.empty(T, HIDDEN, **f32)
        size = int(lib.leat_matmul_workspace(Q6_K, HIDDEN, FFN, T, 0))
        ws = torch.empty(max(size, 1), dtype=torch.uint8, device=device)

        def run(T=T, q=q, d=d, sc=sc, res=res, y=y, ws=ws, size=size):
            if T <= 8:
                _call(lib, "leat_matvec", Q6_K, w["down"].data_ptr(), HIDDEN, FFN, q.data_ptr(), d.data_ptr(),
                      sc.data_ptr(), T, res.data_ptr(), y.data_ptr(), st())  # fmt: skip
            else:
                _call(lib, "leat_matmul", Q6_K, w["down"].data_ptr(), HIDDEN, FFN, q.data_ptr(), d.data_ptr(),
                      sc.data_ptr(), T, res.data_ptr(), y.data_ptr(), ws.data_ptr() if size else None, size, st())  # fmt: skip

        run()
        torch.cuda.synchronize()
        us = _graph_us(torch, run, reps, inner=8)
        wb = nbytes(Q6_K, HIDDEN, FFN)
        out[f"t{T}"] = {"us": round(us, 2), "weight_gbs": round(wb / (us * 1e-6) / 1e9, 1),
                        "tops": round(2 * T * HIDDEN * FFN / (us * 1e-6) / 1e12, 2), "workspace_bytes": size}  # fmt: skip
    out["t16_over_t8"] = round(out["t16"]["us"] / out["t8"]["us"], 3)
    return out


PREFILL_TOKENS = 512
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA


def measure_prefill(torch, lib, w, reps, device):
    """Config 4: 512 tokens x 4096 f32 N(0,1) through the FFN's products on the layer's Q4_K gate
    and up (14336 x 4096) and Q6_K down (4096 x 14336), as leat's feed_forward runs them
    (leat/kernels/matmul.py:1069-1081): norm+quantize, gate+up+GLU on matrix cores writing the
    hidden rows' q8 (quantize_q8's bits), down (+residual). TOPS counts the int8 products'
    2*T*rows*cols ops of the three matrices."""
    T = PREFILL_TOKENS
    f32 = dict(dtype=torch.float32, device=device)
    i32 = dict(dtype=torch.int32, device=device)
    gen = torch.Generator(device=device).manual_seed(4)
    x = torch.randn(T, HIDDEN, generator=gen, **f32)
    norm_w = torch.rand(HIDDEN, generator=gen, **f32) + 0.5
    q8 = {n: (torch.empty(T * n // 4, **i32), torch.empty(T * n // 32, **f32), torch.empty(T * n // 32, **f32))
          for n in (HIDDEN, FFN)}  # fmt: skip
    out = torch.empty(T, HIDDEN, **f32)
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    def quantize(src, n, norm):
        q, d, s = q8[n]
        wp, eps = (norm_w.data_ptr(), 1e-5) if norm else (None, 0.0)
        _call(lib, "leat_quantize_q8", src.data_ptr(), T, n, wp, eps, q.data_ptr(), d.data_ptr(), s.data_ptr(), st())

    def glu():
        # the gated product writing the down product's q8 input itself (no f32 hidden rows)
        xq, xd, xs = q8[HIDDEN]
        hq, hd, hs = q8[FFN]
        _call(lib, "leat_glu_matmul_q8", Q4_K, w["gate"].data_ptr(), w["up"].data_ptr(), FFN, HIDDEN, xq.data_ptr(),
              xd.data_ptr(), xs.data_ptr(), T, 0, None, hq.data_ptr(), hd.data_ptr(), hs.data_ptr(), None, 0, st())  # fmt: skip

    def down():
        hq, hd, hs = q8[FFN]
        _call(lib, "leat_matmul", Q6_K, w["down"].data_ptr(), HIDDEN, FFN, hq.data_ptr(), hd.data_ptr(),
              hs.data_ptr(), T, x.data_ptr(), out.data_ptr(), None, 0, st())  # fmt: skip

    def ffn():
        quantize(x, HIDDEN, True)
        glu()
        down()

    ffn()
    torch.cuda.synchronize()
    ffn_us = _graph_us(torch, ffn, reps)
    glu_us = _graph_us(torch, glu, reps)
    down_us = _graph_us(torch, down, reps)
    glu_ops, down_ops = 2 * T * 2 * FFN * HIDDEN, 2 * T * HIDDEN * FFN
    tops = (glu_ops + down_ops) / (ffn_us * 1e-6) / 1e12
    glu_tops = glu_ops / (glu_us * 1e-6) / 1e12
    return {
        "workload": "512 tokens x 4096: Q4_K gate+up 2x14336x4096 (GLU fused), Q6_K down 4096x14336 (+residual)",
        "ffn_us": round(ffn_us, 1), "glu_us": round(glu_us, 1), "down_us": round(down_us, 1),
        "tops": round(tops, 1), "int8_frac": round(tops / INT8_PEAK_TOPS, 4),
        "down_tops": round(down_ops / (down_us * 1e-6) / 1e12, 1),
        "roofline": {"bound": "mfma", "achieved": glu_tops, "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                     "frac": glu_tops / INT8_PEAK_TOPS, "traffic": None,
                     "kernel": "gate+up GLU matmul (MMQ) with q8 output, Q4_K 2x14336x4096, 512 tokens",
                     "ops_per_launch": glu_ops},
        # matrix-core and VALU busy fractions from rocprofv3 counters (what bounds each kernel)
        "counters": {"glu": profiled_counters("prefill_q4k_glu_q8_512"),
                     "down": profiled_counters("prefill_q6k_residual_512")},
    }  # fmt: skip


# config 5: a Qwen3-30B-A3B-style mixture layer, over as many layers as that model has, so a
# step's chosen experts (24.5 MB a layer at B=1) far exceed the 256 MB MALL
MOE_EXPERTS, MOE_USED, MOE_DIM, MOE_HIDDEN, MOE_LAYERS = 128, 8, 2048, 768, 48
EXPERT_BYTES = 2 * nbytes(Q4_K, MOE_HIDDEN, MOE_DIM) + nbytes(Q6_K, MOE_DIM, MOE_HIDDEN)  # 3,059,712


def measure_moe(torch, lib, B, steps, device, layers):
    """Config 5: the mixture of one token (B=1) or 8 streams (B=8) through 48 layers of 128
    experts (gate and up 768 x 2048 Q4_K, down 2048 x 768 Q6_K, top 8, router logits N(0,1)):
    per layer route, norm+quantize, the chosen experts' gate+up+GLU, quantize (one launch,
    leat_experts_glu_f32), their down (+residual), as leat's mixture on the matrix-vector
    kernels (leat/kernels/experts.py:341-377). Weight bytes are each layer's distinct chosen
    experts, read once each."""
    f32 = dict(dtype=torch.float32, device=device)
    i32 = dict(dtype=torch.int32, device=device)
    gen = torch.Generator(device=device).manual_seed(5)
    P = B * MOE_USED
    scores = [torch.randn(B, MOE_EXPERTS, generator=gen, **f32) for _ in range(MOE_LAYERS)]
    xs = [torch.randn(B, MOE_DIM, generator=gen, **f32) for _ in range(2)]
    norm_w = torch.rand(MOE_DIM, generator=gen, **f32) + 0.5
    ids, weights = torch.empty(P, **i32), torch.empty(P, **f32)
    hq, hd, hs = torch.empty(P * MOE_HIDDEN // 4, **i32), torch.empty(P * MOE_HIDDEN // 32, **f32), torch.empty(P * MOE_HIDDEN // 32, **f32)
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    distinct = []

    def layer(i, w, which="all"):
        x, x_next = xs[i % 2], xs[(i + 1) % 2]
        if which in ("all", "glu"):
            # route, norm + quantize, the chosen experts' gate+up+GLU and its q8 output: one launch
            _call(lib, "leat_experts_glu_f32", Q4_K, w["gate"].data_ptr(), w["up"].data_ptr(), MOE_EXPERTS,
                  MOE_HIDDEN, MOE_DIM, x.data_ptr(), B, norm_w.data_ptr(), 1e-5, scores[i].data_ptr(), MOE_USED,
                  None, None, 0, ids.data_ptr(), weights.data_ptr(), None, hq.data_ptr(), hd.data_ptr(),
                  hs.data_ptr(), st())  # fmt: skip
        if which in ("all", "down"):
            _call(lib, "leat_experts_down", Q6_K, w["down"].data_ptr(), MOE_EXPERTS, MOE_DIM, MOE_HIDDEN,
                  hq.data_ptr(), hd.data_ptr(), hs.data_ptr(), ids.data_ptr(), weights.data_ptr(), B, MOE_USED,
                  None, None, x.data_ptr(), x_next.data_ptr(), st())  # fmt: skip

    for i, w in enumerate(layers):  # eager once: checks every launch, and counts distinct experts
        layer(i, w)
        torch.cuda.synchronize()
        distinct.append(len(set(ids.cpu().tolist())))
    step_us = _graph_us(torch, lambda: [layer(i, w) for i, w in enumerate(layers)], steps)
    # the two expert kernels alone, on the last layer's routing, over every layer's weights
    glu_us = _graph_us(torch, lambda: [layer(i, w, "glu") for i, w in enumerate(layers)], steps) / MOE_LAYERS
    down_us = _graph_us(torch, lambda: [layer(i, w, "down") for i, w in enumerate(layers)], steps) / MOE_LAYERS
    last = distinct[-1]
    step_bytes = sum(distinct) * EXPERT_BYTES
    # the chosen experts' gate and up, the f32 input and scores, the q8 hidden rows written
    glu_bytes = (last * 2 * nbytes(Q4_K, MOE_HIDDEN, MOE_DIM) + B * (MOE_DIM + MOE_EXPERTS) * 4
                 + P * (MOE_HIDDEN + MOE_HIDDEN // 32 * 8))  # fmt: skip
    gbs = step_bytes / (step_us * 1e-6) / 1e9
    glu_gbs = glu_bytes / (glu_us * 1e-6) / 1e9
    moe_traffic, moe_note = profiled_traffic(f"moe_glu_b{B}")
    return {
        "batch": B, "layers": MOE_LAYERS, "distinct_experts_per_layer": round(sum(distinct) / len(distinct), 2),
        "us_per_layer": round(step_us / MOE_LAYERS, 2), "weight_gbs": round(gbs, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "tok_s": round(B * 1e6 / step_us, 1),
        "glu_us": round(glu_us, 2), "down_us": round(down_us, 2),
        "roofline": {"bound": "hbm", "achieved": glu_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": glu_gbs / HBM_PEAK_GBS, "traffic": moe_traffic, "traffic_source": moe_note,
                     "kernel": f"expert gate+up GLU matvec, {last} of 128 experts 2x768x2048 Q4_K, B={B}",
                     "bytes_per_launch": glu_bytes},
    }  # fmt: skip


def moe_layers(torch, device, seed):
    gen = torch.Generator(device=device).manual_seed(seed + 100)
    return [{"gate": synthetic_weights(torch, Q4_K, MOE_EXPERTS * MOE_HIDDEN, MOE_DIM, gen, device),
             "up": synthetic_weights(torch, Q4_K, MOE_EXPERTS * MOE_HIDDEN, MOE_DIM, gen, device),
             "down": synthetic_weights(torch, Q6_K, MOE_EXPERTS * MOE_DIM, MOE_HIDDEN, gen, device)}
            for _ in range(MOE_LAYERS)]  # fmt: skip


def cpu_baseline(budget=20.0):
    """leat's LEAT_KERNELS=ref product (f32 activations, dequantized in ggml's order, f32 sums),
    restated in C with OpenMP (oracle/leat_ref.c), timed on the host: config 1 (a Q8_0 4096 x 4096
    matvec, d = f16(|N| * 0.01), int8 quants uniform in [-127, 127], x N(0, 1)) and one config-2
    layer's 7 matrices at B = 1, each with every thread the process may use and with one; the
    median pass of each, within about `budget` seconds in all."""
    import numpy as np

    from oracle import leat_oracle as O

    path = ROOT / "oracle" / "libleatref.so"
    if not path.exists():
        import subprocess

        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    lib = ctypes.CDLL(str(path))
    lib.leat_ref_linear.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                    ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]  # fmt: skip
    lib.leat_ref_threads.argtypes = [ctypes.c_int]
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    rng = np.random.default_rng(0)
    layer = [(t, r, c, O.matrix_blocks(t, r, c, rng)) for _, t, r, c in MATRICES]
    q8_0 = [(O.Q8_0, 4096, 4096, O.matrix_blocks(O.Q8_0, 4096, 4096, rng))]
    x = {c: rng.standard_normal(c).astype(np.float32) for c in (HIDDEN, FFN)}
    out = np.zeros(FFN, np.float32)

    def timed(mats, seconds):
        times, begin = [], time.perf_counter()
        while True:
            t0 = time.perf_counter()
            for t, r, c, b in mats:
                assert lib.leat_ref_linear(t, b.ctypes.data, r, c, x[c].ctypes.data, 1, out.ctypes.data) == 0
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - begin >= seconds and len(times) >= 3:
                break
        return sorted(times)[len(times) // 2], len(times)

    result = {}
    for threads in (cores, 1):
        lib.leat_ref_threads(threads)
        share = 0.35 if threads > 1 else 0.15
        c1, n1 = timed(q8_0, budget * share * 0.3)
        c2, n2 = timed(layer, budget * share * 0.7)
        result[threads] = {"config1_gbs": round(O.BLOCK[O.Q8_0][1] * 4096 * 4096 / 32 / c1 / 1e9, 2),
                           "config1_ms": round(c1 * 1e3, 3), "config1_passes": n1,
                           "layer_gbs": round(LAYER_BYTES / c2 / 1e9, 2), "layer_ms": round(c2 * 1e3, 2),
                           "layer_passes": n2, "linear_tok_s": round(1.0 / (c2 * LAYERS), 3)}  # fmt: skip
    return {
        "value": result[cores]["layer_gbs"],
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"one config-2 layer's 7 matrices (q,k,v,o,gate,up Q4_K; down Q6_K; {LAYER_BYTES} B) at B=1, "
        "f32 activations, median pass; and config 1, Q8_0 4096x4096 at B=1",
        "all_cores": result[cores],
        "one_core": result[1],
    }


def _leg(r):
    # a config-2 batch size's figures for the JSON line
    return {"weight_gbs": round(r["weight_gbs"], 1), "hbm_frac": round(r["hbm_frac"], 4),
            "linear_tok_s": round(r["linear_tok_s"], 1), "ms_per_step": round(r["ms_per_step"], 4),
            "roofline": r["roofline"]}  # fmt: skip


def measure_peaks(torch, device) -> dict:
    """The rates this GPU reaches, beside the published peaks the rooflines divide by: a plain
    streaming read of 2 GiB (far past the 256 MB MALL; the library's leat_probe_read, 16-byte
    loads, 32 workgroups a CU; the fastest of 3 timings) and back-to-back int8 matrix-core products (leat_probe_mfma_i8:
    4 independent v_mfma_i32_32x32x32_i8 chains a wave, 4 waves a SIMD; the fastest of 3). Each result is checked
    against what the probe must return."""
    from leat_amd import _lib

    nbytes = 2 << 30
    data = torch.ones(nbytes // 4, dtype=torch.int32, device=device)
    groups = 32 * torch.cuda.get_device_properties(device).multi_processor_count
    sink = torch.empty(groups, dtype=torch.int32, device=device)
    # the stream is read at each launch (inside a graph capture it is the capture's own), and the
    # sinks are cleared first, so a replay that ran nothing fails the checks below
    read = lambda: _lib.call("leat_probe_read", data.data_ptr(), nbytes, sink.data_ptr(), groups, _lib.stream())
    sink.zero_()
    read_us = min(_graph_us(torch, read, 10) for _ in range(3))
    if int(sink.to(torch.int64).sum().item()) % (1 << 32) != (nbytes // 4) % (1 << 32):
        raise RuntimeError("probe_read: the word sum is not the buffer's")
    del data
    iters, mfma_groups = 4096, 4 * torch.cuda.get_device_properties(device).multi_processor_count
    msink = torch.empty(4 * mfma_groups, dtype=torch.int32, device=device)
    mfma = lambda: _lib.call("leat_probe_mfma_i8", iters, mfma_groups, msink.data_ptr(), _lib.stream())
    msink.zero_()
    mfma_us = min(_graph_us(torch, mfma, 10) for _ in range(3))
    if not bool((msink == 128 * iters).all().item()):
        raise RuntimeError("probe_mfma_i8: a wave's sums are not 128 x rounds")
    ops = 4 * mfma_groups * iters * 4 * 65536
    return {"hbm_read_gbs": round(nbytes / read_us / 1e3, 1), "hbm_read_bytes": nbytes,
            "int8_mfma_tops": round(ops / mfma_us / 1e6, 1), "int8_mfma_ops": ops,
            "published": {"hbm_gbs": HBM_PEAK_GBS, "int8_tops": INT8_PEAK_TOPS}}  # fmt: skip


def _with_measured_peaks(node, peaks):
    # every roofline of the line gains the measured rate of its bound beside the published peak
    if isinstance(node, dict):
        if node.get("bound") in ("hbm", "mfma") and "peak" in node:
            node["peak_measured"] = peaks["hbm_read_gbs"] if node["bound"] == "hbm" else peaks["int8_mfma_tops"]
        for v in node.values():
            _with_measured_peaks(v, peaks)
    return node


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--legs", default="batches,decode,prefill,moe",
                    help="configurations beside the headline: batches (B=4, 8, 16), decode, prefill, moe")  # fmt: skip
    ap.add_argument("--batches", default="4,8,16", help="the batch sizes of the batches leg")
    ap.add_argument("--moe-batches", default="1,8", help="the batch sizes of the moe leg")
    ap.add_argument("--positions", default="1,4096", help="the cached positions of the decode leg")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also copy 256 MiB device to device: the calibration kernel of HBM byte counters")  # fmt: skip
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build's path runs on a single MI355X, and no "
              "multi-GPU configuration is part of it (see the sharding design).", file=sys.stderr)  # fmt: skip
        sys.exit(2)

    import torch

    from leat_amd import _lib

    lib = _lib.lib()
    device = torch.device("cuda:0")
    gen = torch.Generator(device=device).manual_seed(args.seed)
    layers = [
        {name: synthetic_weights(torch, t, r, c, gen, device) for name, t, r, c in MATRICES}
        for _ in range(LAYERS)
    ]
    torch.cuda.synchronize()
    print(f"weights ready: {LAYERS} layers, {LAYERS * LAYER_BYTES / 1e9:.2f} GB", file=sys.stderr, flush=True)
    b1 = measure(torch, lib, layers, 1, args.steps, args.warmup, device)
    print(f"B=1: {b1['ms_per_step']:.3f} ms/step, {b1['weight_gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    batches = {}
    if "batches" in args.legs:
        for B in (int(b) for b in args.batches.split(",") if b):
            batches[f"b{B}"] = _leg(measure(torch, lib, layers, B, args.steps, args.warmup, device))
            print(f"B={B}: {batches[f'b{B}']['ms_per_step']:.3f} ms/step, {batches[f'b{B}']['weight_gbs']:.0f} GB/s",
                  file=sys.stderr, flush=True)  # fmt: skip
    decode = prefill = moe = None
    if "decode" in args.legs:
        model = decode_model(torch, layers, args.seed, device)
        positions = tuple(int(p) for p in args.positions.split(",") if p)
        decode = measure_decode(torch, model, max(10, args.steps // 2), device, positions)
        print("decode: " + ", ".join(f"P={p} {decode[f'p{p}']['tok_s']:.0f} tok/s" for p in positions)
              + f"; attention {decode['attention']['us']:.1f} us", file=sys.stderr, flush=True)  # fmt: skip
        del model
    if "prefill" in args.legs:
        prefill = measure_prefill(torch, lib, layers[0], max(5, args.steps // 5), device)
        prefill["down_by_tokens"] = measure_few_tokens(torch, lib, layers[0], max(5, args.steps // 5), device)
        print(f"prefill: FFN {prefill['ffn_us']:.0f} us, {prefill['tops']:.0f} TOPS", file=sys.stderr, flush=True)
    del layers
    torch.cuda.empty_cache()
    if "moe" in args.legs:
        experts = moe_layers(torch, device, args.seed)
        moe = {f"b{B}": measure_moe(torch, lib, B, max(5, args.steps // 5), device, experts)
               for B in (int(b) for b in args.moe_batches.split(",") if b)}  # fmt: skip
        print("moe: " + ", ".join(f"{k} {v['us_per_layer']:.1f} us/layer" for k, v in moe.items()),
              file=sys.stderr, flush=True)  # fmt: skip
        del experts
    if args.copy_probe:
        src = torch.ones(64 << 20, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    peaks = measure_peaks(torch, device)
    print(f"peaks: streaming read {peaks['hbm_read_gbs']:.0f} GB/s, int8 matrix cores {peaks['int8_mfma_tops']:.0f} TOPS",
          file=sys.stderr, flush=True)  # fmt: skip
    cpu = None if args.no_cpu else cpu_baseline()
    line = {
        "metric": METRIC,
        "value": round(b1["weight_gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(b1["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "llama3-8b-q4_k_m decode linear layers (config 2 shapes, 32 layers)",
                   "batch": 1, "layers": LAYERS, "weight_bytes_per_step": LAYERS * LAYER_BYTES,
                   "seed": args.seed},  # fmt: skip
        "hbm_frac": round(b1["hbm_frac"], 4),
        "linear_tok_s": round(b1["linear_tok_s"], 1),
        **batches,
        "roofline": b1["roofline"],
        "decode": decode,
        "prefill": prefill,
        "moe": moe,
        "cpu_baseline": cpu,
        "peaks_measured": peaks,
    }
    print(json.dumps(_with_measured_peaks(line, peaks)))


if __name__ == "__main__":
    main()
