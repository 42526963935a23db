"""Benchmark: weight-stream GB/s (% of HBM peak) and decode tok/s of the quantized-weight path,
Llama-3-8B Q4_K_M layer shapes, B = 1 (the headline value) and B = 8.

A step is one decode token's pass over the linear layers of all 32 layers of a random-init
Llama-3-8B-shaped model in Q4_K_M: per layer norm+quantize, q/k/v in one launch, quantize,
o (+residual), norm+quantize, gate+up+SiLU-GLU in one launch, quantize, down (+residual),
exactly as leat's decode step calls them (leat/model.py:497-558 via leat/ops.py:23-55). Weights
are 32 distinct layers of seeded synthetic blocks (4.41 GB, far beyond the 256 MB MALL), resident
in HBM before the timed region; each step is one HIP-graph replay. `value` is weight bytes per
step / step time, as leat's bench counts weight GB/s (leat/bench.py:71-82). The roofline object is
for the dominant kernel (gate+up GLU matvec): a step's 32 launches of it back to back in a HIP
graph, timed with HIP events on their stream; the CPU baseline is the C restatement of leat's
LEAT_KERNELS=ref product (oracle/leat_ref.c) on the host cores, over a bounded sample.

Beside the headline line's decode figures it reports, as sub-objects, the other benchmark
configurations: "prefill" (512 tokens through a layer's FFN on matrix cores, TOPS against the
int8 MFMA peak) and "moe" (a Qwen3-30B-A3B-style mixture at B = 1 and 8, weight GB/s of the
distinct chosen experts), each with the roofline of its dominant kernel.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--seed S] [--no-cpu] [--legs prefill,moe]
                    [--copy-probe]
"""

from __future__ import annotations

import argparse
import ctypes
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
    return {
        "ms_per_step": ms,
        "weight_gbs": gbs,
        "hbm_frac": gbs / HBM_PEAK_GBS,
        "tok_s": B * 1000.0 / ms,
        "glu_us": glu_us,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": profiled_traffic(GLU_KERNELS.get(B, "")),
                     "traffic_source": "profiles/decode_linear_hbm_bytes.md (rocprofv3 FETCH_SIZE, WRITE_SIZE)",
                     "kernel": f"gate+up GLU matvec, Q4_K 2x14336x4096, B={B}"
                               + (" (quantizes its f32 input and its output)" if B <= 2 else ""),
                     "bytes_per_launch": glu_bytes(B)},  # fmt: skip
    }


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "decode_linear_hbm_bytes.md")


def profiled_traffic(kernel: str):
    """HBM bytes per dispatch of `kernel` as the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    records them (calibrated against a copy of known size), or None if it does not."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(r"^" + re.escape(kernel) + r" (\d+)$", text, re.M)
    return int(m.group(1)) if m else None


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


# the GLU kernels of the decode legs, as rocprofv3 names them
GLU_KERNELS = {1: "rows_kernel<12, 1, 2, 4, 8, 2, true, true>", 8: "tiles_kernel<12, 2, 4>"}

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
    return {
        "batch": B, "layers": MOE_LAYERS, "distinct_experts_per_layer": round(sum(distinct) / len(distinct), 2),
        "us_per_layer": round(step_us / MOE_LAYERS, 2), "weight_gbs": round(gbs, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "tok_s": round(B * 1e6 / step_us, 1),
        "glu_us": round(glu_us, 2), "down_us": round(down_us, 2),
        "roofline": {"bound": "hbm", "achieved": glu_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": glu_gbs / HBM_PEAK_GBS, "traffic": None,
                     "kernel": f"expert gate+up GLU matvec, {last} of 128 experts 2x768x2048 Q4_K, B={B}",
                     "bytes_per_launch": glu_bytes},
    }  # fmt: skip


def moe_layers(torch, device, seed):
    gen = torch.Generator(device=device).manual_seed(seed + 100)
    return [{"gate": synthetic_weights(torch, Q4_K, MOE_EXPERTS * MOE_HIDDEN, MOE_DIM, gen, device),
             "up": synthetic_weights(torch, Q4_K, MOE_EXPERTS * MOE_HIDDEN, MOE_DIM, gen, device),
             "down": synthetic_weights(torch, Q6_K, MOE_EXPERTS * MOE_DIM, MOE_HIDDEN, gen, device)}
            for _ in range(MOE_LAYERS)]  # fmt: skip


def cpu_baseline(seconds=10.0, cap=30.0):
    """leat's LEAT_KERNELS=ref product (f32 activations, dequantize in ggml's order, f32 sums),
    restated in C with OpenMP, over one synthetic layer's 7 matrices at B=1, repeated for about
    `seconds` (at most `cap`): weight GB/s, the median layer pass."""
    import numpy as np

    from oracle import leat_oracle as O

    path = ROOT / "oracle" / "libleatref.so"
    if not path.exists():
        import subprocess

        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    lib = ctypes.CDLL(str(path))
    lib.leat_ref_linear.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                    ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]  # fmt: skip
    rng = np.random.default_rng(0)
    mats = [(t, r, c, O.matrix_blocks(t, r, c, rng)) for _, t, r, c in MATRICES]
    x = {c: rng.standard_normal(c).astype(np.float32) for c in (HIDDEN, FFN)}
    out = np.zeros(FFN, np.float32)
    times, begin = [], time.perf_counter()
    while True:
        t0 = time.perf_counter()
        for t, r, c, b in mats:
            assert lib.leat_ref_linear(t, b.ctypes.data, r, c, x[c].ctypes.data, 1, out.ctypes.data) == 0
        times.append(time.perf_counter() - t0)
        elapsed = time.perf_counter() - begin
        if (elapsed >= seconds and len(times) >= 5) or elapsed >= cap:
            break
    per_layer = sorted(times)[len(times) // 2]
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {
        "value": LAYER_BYTES / per_layer / 1e9,
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"one Llama-3-8B layer's 7 matrices (q,k,v,o,gate,up Q4_K; down Q6_K; {LAYER_BYTES} B) "
        f"at B=1, f32 activations, {len(times)} passes in {time.perf_counter() - begin:.1f} s, median",
        "tok_s_equiv": 1.0 / (per_layer * LAYERS),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--legs", default="prefill,moe", help="configurations beside decode: prefill, moe")
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
    b8 = measure(torch, lib, layers, 8, args.steps, args.warmup, device)
    print(f"B=8: {b8['ms_per_step']:.3f} ms/step, {b8['weight_gbs']:.0f} GB/s", file=sys.stderr, flush=True)
    prefill = moe = None
    if "prefill" in args.legs:
        prefill = measure_prefill(torch, lib, layers[0], max(5, args.steps // 5), device)
        print(f"prefill: FFN {prefill['ffn_us']:.0f} us, {prefill['tops']:.0f} TOPS", file=sys.stderr, flush=True)
    del layers
    torch.cuda.empty_cache()
    if "moe" in args.legs:
        experts = moe_layers(torch, device, args.seed)
        moe = {f"b{B}": measure_moe(torch, lib, B, max(5, args.steps // 5), device, experts) for B in (1, 8)}
        print(f"moe: B=1 {moe['b1']['us_per_layer']:.1f} us/layer, B=8 {moe['b8']['us_per_layer']:.1f} us/layer",
              file=sys.stderr, flush=True)  # fmt: skip
        del experts
    if args.copy_probe:
        src = torch.ones(64 << 20, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
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
        "tok_s": round(b1["tok_s"], 1),
        "b8": {"weight_gbs": round(b8["weight_gbs"], 1), "hbm_frac": round(b8["hbm_frac"], 4),
               "tok_s": round(b8["tok_s"], 1), "ms_per_step": round(b8["ms_per_step"], 4),
               "roofline": b8["roofline"]},  # fmt: skip
        "roofline": b1["roofline"],
        "prefill": prefill,
        "moe": moe,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
