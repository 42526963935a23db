"""A Llama-architecture decoder on this library's kernels: the part of leat's model
(leat/model.py:370-423, 497-558) a Llama 3.1 8B decode step runs.

Per step and row (one token of one sequence each): the token's embedding; per layer RMSNorm and
q/k/v in one launch that quantizes its own input, RoPE with the keys and values stored in an f16
cache, FlashDecoding over the row's slot, o plus the residual, the feed-forward block (norm, gate
and up with SiLU in one launch writing the down product's int8 input, down plus the residual);
the final norm and the Q6_K output head in one launch; the greedy next token. Every launch takes
device buffers and device slots and positions, so a step is captured once as a HIP graph and
replayed (leat/engine.py:784-806 captures its steps the same way with TinyJit).

Weights are GGUF blocks as stored (QTensor); `synthetic` draws a random-init model of a given
shape in Q4_K_M (Q4_K matrices, Q6_K down and output) with the benchmark's distributions.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from leat_amd import kernels, ops
from leat_amd.quant import BLOCK, GGMLType, QTensor


@dataclass(frozen=True)
class LlamaConfig:
    """The sizes of a Llama-architecture model (leat/model.py's Config for arch "llama")."""

    dim: int = 4096
    layers: int = 32
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 14336
    vocab: int = 128256
    norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    # Llama 3.1's frequency scaling (factor, low and high frequency factors, original context),
    # which GGUF files carry as rope_freqs.weight; None for plain RoPE
    rope_scaling: tuple[float, float, float, int] | None = (8.0, 1.0, 4.0, 8192)
    context: int = 4096  # cache positions per slot
    slots: int = 1  # sequences the cache holds


LLAMA3_8B = LlamaConfig()


def llama3_rope_factors(dims: int, theta: float, scaling: tuple[float, float, float, int]) -> list[float]:
    """What divides each RoPE frequency under Llama 3.1's scaling, as its GGUF's rope_freqs holds
    (Meta's published rule): wavelengths below original / high stay (1), above original / low
    are scaled by `factor`, and between them the two blend linearly in original / wavelength."""
    factor, low, high, original = scaling
    out = []
    for i in range(dims // 2):
        wavelength = 2 * math.pi * theta ** (2 * i / dims)  # of frequency theta^(-2i/d)
        if wavelength < original / high:
            out.append(1.0)
        elif wavelength > original / low:
            out.append(factor)
        else:
            smooth = (original / wavelength - low) / (high - low)
            out.append(1.0 / ((1 - smooth) / factor + smooth))
    return out


def rope_table(dims: int, theta: float, length: int, factors: list[float] | None, device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos and sin (length, dims / 2) f32 of angle pos * theta^(-2i/d) / factor_i, the angle in f32
    as leat computes it (leat/model.py:688-723, plain RoPE without YaRN), cos and sin of that f32
    angle rounded to f32."""
    freqs = torch.tensor([theta ** (-2 * i / dims) for i in range(dims // 2)], dtype=torch.float32)
    angles = torch.arange(length, dtype=torch.float32).unsqueeze(1) * freqs.unsqueeze(0)
    if factors is not None:
        angles = angles / torch.tensor(factors, dtype=torch.float32).unsqueeze(0)
    wide = angles.double()
    return torch.cos(wide).float().to(device), torch.sin(wide).float().to(device)


@dataclass
class Layer:
    attn_norm: torch.Tensor
    q: QTensor
    k: QTensor
    v: QTensor
    o: QTensor
    ffn_norm: torch.Tensor
    gate: QTensor
    up: QTensor
    down: QTensor


@dataclass
class Weights:
    embed: QTensor
    layers: list[Layer]
    output_norm: torch.Tensor
    output: QTensor


def _synthetic_blocks(ggml_type: GGMLType, rows: int, cols: int, gen: torch.Generator, device) -> QTensor:
    # uniform bytes, then Q4_K d = f16(|N| * 0.002), dmin = f16(|N| * 0.001); Q6_K d = f16(|N| * 0.002)
    elements, size = BLOCK[ggml_type]
    n = rows * cols // elements
    blocks = torch.randint(0, 256, (n, size), dtype=torch.uint8, device=device, generator=gen)

    def f16(scale: float) -> torch.Tensor:
        return (torch.randn(n, device=device, generator=gen).abs() * scale).half().view(torch.uint8).view(n, 2)

    if ggml_type == GGMLType.Q4_K:
        blocks[:, 0:2] = f16(0.002)
        blocks[:, 2:4] = f16(0.001)
    elif ggml_type == GGMLType.Q6_K:
        blocks[:, 208:210] = f16(0.002)
    else:
        raise NotImplementedError(ggml_type)
    return QTensor(blocks, ggml_type, (rows, cols))


def synthetic(config: LlamaConfig, seed: int = 0, device="cuda") -> Weights:
    """A random-init model of `config` in Q4_K_M: Q4_K embedding, attention and gate/up, Q6_K down
    and output head, norm weights uniform in [0.5, 1.5)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    c, q4, q6 = config, GGMLType.Q4_K, GGMLType.Q6_K

    def norm() -> torch.Tensor:
        return torch.rand(c.dim, generator=gen, device=device) + 0.5

    layers = [
        Layer(norm(), _synthetic_blocks(q4, c.heads * c.head_dim, c.dim, gen, device),
              _synthetic_blocks(q4, c.kv_heads * c.head_dim, c.dim, gen, device),
              _synthetic_blocks(q4, c.kv_heads * c.head_dim, c.dim, gen, device),
              _synthetic_blocks(q4, c.dim, c.heads * c.head_dim, gen, device), norm(),
              _synthetic_blocks(q4, c.ffn, c.dim, gen, device), _synthetic_blocks(q4, c.ffn, c.dim, gen, device),
              _synthetic_blocks(q6, c.dim, c.ffn, gen, device))
        for _ in range(c.layers)
    ]  # fmt: skip
    embed = _synthetic_blocks(q4, c.vocab, c.dim, gen, device)
    return Weights(embed, layers, norm(), _synthetic_blocks(q6, c.vocab, c.dim, gen, device))


def from_gguf(path, context: int = 4096, slots: int = 1, device="cuda") -> Model:
    """A Llama-architecture model from a GGUF file (leat/gguf.py's reader, leat/model.py's
    names for arch "llama"): the sizes from its llama.* metadata, the matrices from its tensors in
    one transfer, Llama 3.1's RoPE factors from rope_freqs.weight where the file has them."""
    from leat_amd.gguf import GGUF

    g = GGUF.open(path)
    m = g.metadata
    arch = m.get("general.architecture", "llama")
    if arch != "llama":
        raise ValueError(f"{path}: architecture {arch!r}; this decoder runs llama")
    dim, heads = int(m["llama.embedding_length"]), int(m["llama.attention.head_count"])
    layers = int(m["llama.block_count"])
    names = ["token_embd.weight", "output_norm.weight", "output.weight"]
    for i in range(layers):
        names += [f"blk.{i}.{n}.weight" for n in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm",
                                                     "ffn_gate", "ffn_up", "ffn_down")]  # fmt: skip
    if "rope_freqs.weight" in g.tensors:
        names.append("rope_freqs.weight")
    t = g.load(device, names)
    vocab = t["token_embd.weight"].shape[0]
    config = LlamaConfig(
        dim=dim, layers=layers, heads=heads, kv_heads=int(m.get("llama.attention.head_count_kv", heads)),
        head_dim=dim // heads, ffn=int(m["llama.feed_forward_length"]), vocab=vocab,
        norm_eps=float(m.get("llama.attention.layer_norm_rms_epsilon", 1e-5)),
        rope_theta=float(m.get("llama.rope.freq_base", 10000.0)), rope_scaling=None, context=context, slots=slots,
    )  # fmt: skip

    def norm(name: str) -> torch.Tensor:
        return t[name].dequant()

    built = [Layer(norm(f"blk.{i}.attn_norm.weight"), t[f"blk.{i}.attn_q.weight"], t[f"blk.{i}.attn_k.weight"],
                   t[f"blk.{i}.attn_v.weight"], t[f"blk.{i}.attn_output.weight"], norm(f"blk.{i}.ffn_norm.weight"),
                   t[f"blk.{i}.ffn_gate.weight"], t[f"blk.{i}.ffn_up.weight"], t[f"blk.{i}.ffn_down.weight"])
             for i in range(layers)]  # fmt: skip
    weights = Weights(t["token_embd.weight"], built, norm("output_norm.weight"), t["output.weight"])
    factors = t["rope_freqs.weight"].dequant().cpu().tolist() if "rope_freqs.weight" in t else None
    device_of = t["output.weight"].data.device
    return Model(config, weights, rope=rope_table(config.head_dim, config.rope_theta, context, factors, device_of))


def weight_bytes(w: Weights) -> int:
    """The bytes of matrices a decode step streams: every layer's, and the output head."""
    per_layer = sum(m.nbytes for layer in w.layers for m in (layer.q, layer.k, layer.v, layer.o, layer.gate, layer.up, layer.down))
    return per_layer + w.output.nbytes


@dataclass
class Model:
    """A decoder with its f16 KV cache (one (2, slots, kv_heads, context, head_dim) tensor per
    layer) and RoPE tables."""

    config: LlamaConfig
    weights: Weights
    cache: list[torch.Tensor] = field(default_factory=list)
    rope: tuple[torch.Tensor, torch.Tensor] | None = None
    _workspaces: dict[int, torch.Tensor] = field(default_factory=dict, repr=False)

    def __post_init__(self):
        c = self.config
        device = self.weights.output.data.device
        if not self.cache:
            self.cache = [torch.zeros(2, c.slots, c.kv_heads, c.context, c.head_dim, dtype=torch.float16, device=device)
                          for _ in range(c.layers)]  # fmt: skip
        if self.rope is None:
            factors = None if c.rope_scaling is None else llama3_rope_factors(c.head_dim, c.rope_theta, c.rope_scaling)
            self.rope = rope_table(c.head_dim, c.rope_theta, c.context, factors, device)

    def _attention_workspace(self, rows: int) -> torch.Tensor | None:
        # one workspace for every layer's attention of a decode batch, kept for the model's
        # life (a captured step replays with it); long prompt chunks get theirs per call
        if rows > 64 or ops.reference_mode() or not self.weights.output.data.is_cuda:
            return None
        if rows not in self._workspaces:
            c = self.config
            self._workspaces[rows] = kernels.attention_workspace(rows, c.heads, c.context, self.weights.output.data.device)
        return self._workspaces[rows]

    def logits(self, tokens: torch.Tensor, slots: torch.Tensor, positions: torch.Tensor,
               lengths: torch.Tensor | None = None, last: bool = False,
               max_length: int | None = None) -> torch.Tensor:  # fmt: skip
        """One step of `tokens` (B,) int32, row b the token of the sequence in cache slot slots[b]
        at position positions[b] (device tensors): the logits (B, vocab) f32. Row b's keys and
        values go to its slot at its position, and it attends over positions 0..positions[b]
        (lengths, positions + 1, may be given to save the addition). Rows of one sequence's
        consecutive positions are a chunk of its prompt, each row seeing those before it; with
        `last`, only the last row's logits are computed, (1, vocab). `max_length`, if given, bounds
        every row's length (the context otherwise): it sizes the attention launches."""
        c, w = self.config, self.weights
        B = tokens.shape[0]
        if lengths is None:
            lengths = positions + 1
        x = ops.embedding(tokens, w.embed).view(1, B, c.dim)
        scale = 1.0 / math.sqrt(c.head_dim)
        rope = (self.rope, c.head_dim)
        longest = c.context if max_length is None else int(max_length)
        for layer, cache in zip(w.layers, self.cache, strict=True):
            q_rot = ops.qkv_rotate(x, layer.q, layer.k, layer.v, (layer.attn_norm, c.norm_eps), cache, None, rope, False,
                                   slots, positions)  # fmt: skip
            x = ops.attention_linear(q_rot, cache, None, scale, layer.o, x, slots, lengths, longest,
                                     self._attention_workspace(B))  # fmt: skip
            x = ops.feed_forward(x, layer.gate, layer.up, layer.down, (layer.ffn_norm, c.norm_eps))
        if last:
            x, B = x[:, -1:], 1
        (logits,) = ops.linears(x, w.output, norm=(w.output_norm, c.norm_eps))
        return logits.view(B, c.vocab)

    def step(self, tokens: torch.Tensor, slots: torch.Tensor, positions: torch.Tensor,
             lengths: torch.Tensor | None = None, last: bool = False,
             max_length: int | None = None) -> torch.Tensor:  # fmt: skip
        """The greedy next token of each row (of the last only, with `last`): argmax of logits(),
        (B,) int32."""
        return ops.argmax(self.logits(tokens, slots, positions, lengths, last, max_length)).view(-1)


# the keys FlashDecoding takes in one chunk for launches of at most this many keys (8 waves of 16
# keys, attention.hip): a step whose rows are all this short runs no combine pass, and its partial
# kernel one chunk a row
SHORT_CONTEXT = 128


class GraphStep:
    """A decode step of B rows captured as HIP graphs over static device buffers `tokens`, `slots`
    and `positions` (B,) int32, which the caller fills before replaying (building the graphs
    writes nothing to the cache); replay() runs a step on whatever the buffers hold and leaves the
    next tokens in `next`. With `advance`, the graph also moves each row on: tokens = next,
    positions += 1, so replays decode one token after another with no host work between them.

    One graph is captured per length bucket (`buckets`, by default SHORT_CONTEXT, and always the
    context), each sizing its attention launches for rows of at most that many keys: a caller
    that knows its rows' longest length (position + 1) passes it to replay(), which runs the
    smallest graph that covers it; without it the context's graph runs."""

    def __init__(self, model: Model, batch: int, advance: bool = True, buckets: tuple[int, ...] = (SHORT_CONTEXT,)):
        device = model.weights.output.data.device
        context = model.config.context
        self.model, self.batch = model, batch
        self.buckets = tuple(sorted({min(int(b), context) for b in buckets if int(b) > 0} | {context}))
        self.tokens = torch.zeros(batch, dtype=torch.int32, device=device)
        self.slots = torch.zeros(batch, dtype=torch.int32, device=device)
        # past the cache's positions: the eager warm-up below stores no key or value anywhere
        self.positions = torch.full((batch,), context, dtype=torch.int32, device=device)
        self.lengths = torch.ones(batch, dtype=torch.int32, device=device)
        for longest in self.buckets:  # once eagerly: every launch checked, and the memory pool warmed
            self._run(False, longest)
        torch.cuda.synchronize(device)
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self._next: dict[int, torch.Tensor] = {}
        for longest in self.buckets:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._next[longest] = self._run(advance, longest)
            self._graphs[longest] = graph
        self.graph = self._graphs[context]
        self.next = self._next[context]

    def _run(self, advance: bool, longest: int) -> torch.Tensor:
        torch.add(self.positions, 1, out=self.lengths)
        nxt = self.model.step(self.tokens, self.slots, self.positions, self.lengths, max_length=longest)
        if advance:
            self.tokens.copy_(nxt)
            self.positions.add_(1)
        return nxt

    def replay(self, max_length: int | None = None) -> None:
        """One step; `max_length`, if given, is at least every row's length (position + 1) in this
        step, and selects the smallest graph whose bucket covers it."""
        longest = self.buckets[-1]
        if max_length is not None:
            if max_length > longest:
                raise ValueError(f"rows of {max_length} keys in a context of {longest}")
            longest = next(b for b in self.buckets if b >= max_length)
        self._graphs[longest].replay()
        self.next = self._next[longest]
