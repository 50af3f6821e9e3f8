"""A full decode step through the vLLM backend path, without vLLM (config 5).

A random-init decoder of the Qwen3-4B shape (36 layers, hidden 2560, 32 query
/ 8 kv heads of 128, SwiGLU 9728, RMSNorm with per-head q/k norms, rotary
positions, tied embeddings, bf16) runs one token per sequence per step. Each
layer's attention goes through the same two calls the backend makes inside
vLLM: ``kv_cache_update`` (the backend's ``do_kv_cache_update``, the HIP
``reshape_and_cache`` page append at ``slot_mapping``) and ``forward_decode``
(the backend's ``forward``: vLLM metadata -> ``flash_attn_with_kvcache`` ->
the ``mi355x_split_decode`` kernels). The metadata object carries the fields
vLLM's FlashAttention metadata carries for decode.

As vLLM does for decode, a whole step (all layers and the logits) is captured
once in a HIP graph and replayed (``eager=True``: every step launched from
Python instead, vLLM's ``enforce_eager``); between replays the host-side model runner
advances the metadata (lengths, slots, positions) and picks the next tokens
greedily. The prompt part of the KV cache is synthetic (random K/V, no
prefill run): the decode step reads it exactly as it would read a real one.

Run: ``python -m mxflashattn_amd.integrations.vllm.decode_step`` (one JSON line).
"""

from __future__ import annotations

import argparse
import json
import math
import sys
from dataclasses import dataclass

import torch

from .decoder_adapter import forward_decode, kv_cache_update


@dataclass(frozen=True)
class DecoderShape:
    layers: int = 36
    hidden: int = 2560
    q_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 9728
    vocab: int = 151936
    rope_theta: float = 1.0e6
    eps: float = 1.0e-6


QWEN3_4B = DecoderShape()


@dataclass
class DecodeMetadata:
    """The fields of vLLM's FlashAttention metadata the decode path reads."""

    num_actual_tokens: int
    max_query_len: int
    query_start_loc: torch.Tensor
    max_seq_len: int
    seq_lens: torch.Tensor      # int32 [B], including the token being decoded
    block_table: torch.Tensor   # int32 [B, W]
    slot_mapping: torch.Tensor  # int64 [B], cache slot of the token being decoded
    use_cascade: bool = False
    scheduler_metadata: torch.Tensor | None = None
    causal: bool = True


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return torch.nn.functional.rms_norm(x, (x.shape[-1],), weight, eps)


class DecoderModel:
    """Random-init weights of ``shape``; ``step`` runs one decode token per sequence."""

    def __init__(self, shape: DecoderShape, device: torch.device, dtype=torch.bfloat16,
                 seed: int = 20261007, kv_cache_dtype: str = "auto") -> None:
        self.shape = shape
        self.device = device
        self.dtype = dtype
        # vLLM's cache dtype string: "auto" (the model dtype) or "fp8" (e4m3fn
        # with per-tensor scales, here 1.0 as a float32 device scalar per layer).
        self.kv_cache_dtype = kv_cache_dtype
        self.k_scale = torch.ones(1, device=device, dtype=torch.float32)
        self.v_scale = torch.ones(1, device=device, dtype=torch.float32)
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        s = shape

        def w(*dims, std=0.02):
            return (torch.randn(*dims, generator=g, device=device, dtype=torch.float32) * std
                    ).to(dtype)

        qkv_out = (s.q_heads + 2 * s.kv_heads) * s.head_dim
        self.embed = w(s.vocab, s.hidden)
        self.layers = []
        for _ in range(s.layers):
            self.layers.append({
                "ln1": torch.ones(s.hidden, device=device, dtype=dtype),
                "qkv": w(qkv_out, s.hidden),
                "q_norm": torch.ones(s.head_dim, device=device, dtype=dtype),
                "k_norm": torch.ones(s.head_dim, device=device, dtype=dtype),
                "o": w(s.hidden, s.q_heads * s.head_dim),
                "ln2": torch.ones(s.hidden, device=device, dtype=dtype),
                "gate_up": w(2 * s.intermediate, s.hidden),
                "down": w(s.hidden, s.intermediate),
            })
        self.final_norm = torch.ones(s.hidden, device=device, dtype=dtype)
        self.inv_freq = 1.0 / (s.rope_theta ** (
            torch.arange(0, s.head_dim, 2, device=device, dtype=torch.float32) / s.head_dim))
        self.scale = s.head_dim ** -0.5

    def weight_bytes(self) -> int:
        n = self.embed.numel() + self.final_norm.numel()
        for layer in self.layers:
            n += sum(t.numel() for t in layer.values())
        return n * self.embed.element_size()

    def rope_tables(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """cos/sin [B, 1, head_dim] of the step's positions (shared by all layers)."""
        freqs = positions.float()[:, None] * self.inv_freq[None, :]      # [B, HD/2]
        emb = torch.cat([freqs, freqs], dim=-1)[:, None, :]
        return emb.cos(), emb.sin()

    @staticmethod
    def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        """Rotary positions (rotate-half form) on [B, heads, head_dim], in fp32."""
        xf = x.float()
        half = xf.shape[-1] // 2
        rotated = torch.cat([-xf[..., half:], xf[..., :half]], dim=-1)
        return (xf * cos + rotated * sin).to(x.dtype)

    def attention(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  kv_cache: torch.Tensor, meta: DecodeMetadata, out: torch.Tensor) -> None:
        """The two backend calls vLLM makes per layer: cache update, then decode."""
        kv_cache_update(k, v, kv_cache, meta.slot_mapping, self.kv_cache_dtype, self.k_scale,
                        self.v_scale)
        forward_decode(q, kv_cache, meta, out, softmax_scale=self.scale,
                       kv_cache_dtype=self.kv_cache_dtype, k_scale=self.k_scale,
                       v_scale=self.v_scale)

    def step(self, tokens: torch.Tensor, positions: torch.Tensor, kv_caches: list[torch.Tensor],
             meta: DecodeMetadata) -> torch.Tensor:
        """One decode token for each of the B sequences; returns logits [B, vocab]."""
        s = self.shape
        bsz = tokens.shape[0]
        nq, nkv = s.q_heads * s.head_dim, s.kv_heads * s.head_dim
        x = self.embed[tokens]
        cos, sin = self.rope_tables(positions)
        attn_out = torch.empty(bsz, nq, device=self.device, dtype=self.dtype)
        for i, layer in enumerate(self.layers):
            h = rms_norm(x, layer["ln1"], s.eps)
            qkv = h @ layer["qkv"].t()
            q = qkv[:, :nq].view(bsz, s.q_heads, s.head_dim)
            k = qkv[:, nq:nq + nkv].view(bsz, s.kv_heads, s.head_dim)
            v = qkv[:, nq + nkv:].view(bsz, s.kv_heads, s.head_dim)
            q = self.rope(rms_norm(q, layer["q_norm"], s.eps), cos, sin)
            k = self.rope(rms_norm(k, layer["k_norm"], s.eps), cos, sin)
            self.attention(i, q, k, v, kv_caches[i], meta, attn_out)
            x = x + attn_out @ layer["o"].t()
            h = rms_norm(x, layer["ln2"], s.eps)
            gate, up = (h @ layer["gate_up"].t()).chunk(2, dim=-1)
            x = x + (torch.nn.functional.silu(gate) * up) @ layer["down"].t()
        x = rms_norm(x, self.final_norm, s.eps)
        return x @ self.embed.t()


@dataclass
class DecodeState:
    """Static buffers of the captured step and the host-side runner state."""

    tokens: torch.Tensor     # int64 [B]
    positions: torch.Tensor  # int64 [B], position of the token being decoded
    kv_caches: list[torch.Tensor]
    meta: DecodeMetadata
    prompt_lens: torch.Tensor  # int64 [B] (host)
    page_size: int


def lognormal_prompt_lengths(batch: int, median: int, sigma: float, lo: int, hi: int,
                             seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(batch, generator=g, dtype=torch.float64)
    return torch.exp(math.log(median) + sigma * z).round().clamp(lo, hi).to(torch.int64)


def build_state(model: DecoderModel, batch: int, prompt_lens: torch.Tensor, new_tokens: int,
                page_size: int = 16, seed: int = 20261007) -> DecodeState:
    """Paged KV caches holding a synthetic prompt for every sequence, with pages
    for the prompt plus ``new_tokens`` decoded tokens from a shuffled pool."""
    s = model.shape
    dev = model.device
    pages_per_seq = ((prompt_lens + new_tokens + page_size - 1) // page_size).tolist()
    width = max(pages_per_seq)
    total = sum(pages_per_seq)
    g = torch.Generator().manual_seed(seed + 1)
    perm = torch.randperm(total, generator=g)
    table = torch.zeros(batch, width, dtype=torch.int32)
    start = 0
    for b, n in enumerate(pages_per_seq):
        table[b, :n] = perm[start:start + n].to(torch.int32)
        start += n
    gd = torch.Generator(device=dev)
    gd.manual_seed(seed + 2)
    kv_caches = []
    fp8 = model.kv_cache_dtype.startswith("fp8")
    for _ in range(s.layers):
        cache = torch.empty(2, total, page_size, s.kv_heads, s.head_dim, device=dev,
                            dtype=model.dtype)
        cache.normal_(generator=gd)
        if fp8:  # N(0, 1) values are well inside e4m3fn's range
            cache = cache.to(torch.float8_e4m3fn)
        kv_caches.append(cache)
    table = table.to(dev)
    seq_lens = prompt_lens.to(dev, torch.int32)  # lengths before the first decoded token
    meta = DecodeMetadata(
        num_actual_tokens=batch, max_query_len=1,
        query_start_loc=torch.arange(batch + 1, device=dev, dtype=torch.int32),
        max_seq_len=int(prompt_lens.max()) + new_tokens, seq_lens=seq_lens,
        block_table=table, slot_mapping=torch.zeros(batch, device=dev, dtype=torch.int64))
    tokens = torch.randint(0, s.vocab, (batch,), generator=gd, device=dev)
    state = DecodeState(tokens=tokens, positions=torch.zeros(batch, device=dev,
                                                             dtype=torch.int64),
                        kv_caches=kv_caches, meta=meta, prompt_lens=prompt_lens,
                        page_size=page_size)
    advance(state)
    return state


def advance(state: DecodeState) -> None:
    """Model-runner update before a step: the token being decoded sits at
    position = current length; its slot comes from the block table; the
    lengths then include it (vLLM writes the token before attention)."""
    meta, ps = state.meta, state.page_size
    pos = meta.seq_lens.to(torch.int64)
    state.positions.copy_(pos)
    page = meta.block_table.gather(1, (pos // ps)[:, None]).squeeze(1).to(torch.int64)
    meta.slot_mapping.copy_(page * ps + pos % ps)
    meta.seq_lens.add_(1)


def run(batch: int = 128, new_tokens: int = 256, shape: DecoderShape = QWEN3_4B,
        median: int = 1024, sigma: float = 1.0, lo: int = 16, hi: int = 8192,
        page_size: int = 16, device: torch.device | None = None, seed: int = 20261007,
        kv_cache_dtype: str = "auto", eager: bool = False) -> dict:
    """Decode ``new_tokens`` tokens for ``batch`` sequences; timing and share.

    eager: every step is launched from Python (vLLM's ``enforce_eager=True``,
    the mode of the reference's end-to-end runs) instead of replaying a
    captured HIP graph."""
    device = device or torch.device("cuda", torch.cuda.current_device())
    model = DecoderModel(shape, device, seed=seed, kv_cache_dtype=kv_cache_dtype)
    prompt = lognormal_prompt_lengths(batch, median, sigma, lo, hi, seed)
    state = build_state(model, batch, prompt, new_tokens, page_size, seed)
    stream = torch.cuda.Stream(device)
    if eager:
        return _run_eager(model, state, batch, new_tokens, shape, prompt, stream,
                          kv_cache_dtype, (median, sigma, lo, hi))

    def step():
        return model.step(state.tokens, state.positions, state.kv_caches, state.meta)

    # Eager warm-up on the capture stream (allocates the decode workspace there),
    # then capture one step. Warm-up and capture write the token at the same
    # slots, so the cache content is unchanged by them.
    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        logits = step()

    # Attention alone: the same cache updates and decode calls for every layer.
    q_static = torch.randn(batch, shape.q_heads, shape.head_dim, device=device,
                           dtype=model.dtype)
    kv_static = torch.randn(batch, shape.kv_heads, shape.head_dim, device=device,
                            dtype=model.dtype)
    attn_static = torch.empty(batch, shape.q_heads * shape.head_dim, device=device,
                              dtype=model.dtype)
    attn_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(attn_graph, stream=stream):
        for i in range(shape.layers):
            model.attention(i, q_static, kv_static, kv_static, state.kv_caches[i], state.meta,
                            attn_static)

    steps = new_tokens - 1  # the first token's slots were used by warm-up and capture
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        graph.replay()  # the first decoded token
        state.tokens.copy_(logits.argmax(-1))
        start.record(stream)
        for _ in range(steps):
            advance(state)
            graph.replay()
            state.tokens.copy_(logits.argmax(-1))
        end.record(stream)
    torch.cuda.synchronize()
    step_ms = start.elapsed_time(end) / steps

    # Attention share: the attention-only graph replayed at the final lengths.
    reps = 20
    a0 = torch.cuda.Event(enable_timing=True)
    a1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        attn_graph.replay()
        a0.record(stream)
        for _ in range(reps):
            attn_graph.replay()
        a1.record(stream)
    torch.cuda.synchronize()
    attn_ms = a0.elapsed_time(a1) / reps
    final_lens = state.meta.seq_lens.to(torch.int64)
    # K and V bytes the attention calls read per step, over all layers.
    kv_bytes_step = (int(final_lens.sum().item()) * shape.kv_heads * shape.head_dim * 2
                     * state.kv_caches[0].element_size() * shape.layers)
    finite = bool(torch.isfinite(logits.float()).all().item())
    del graph, attn_graph
    return {
        "decode_tok_s": round(batch / (step_ms * 1e-3), 1),
        "step_ms": round(step_ms, 4),
        "attention_ms": round(attn_ms, 4),
        "attention_share": round(attn_ms / step_ms, 4),
        "attention_kv_gb_s": round(kv_bytes_step / (attn_ms * 1e-3) / 1e9, 1),
        "batch": batch,
        "kv_cache_dtype": "fp8_e4m3" if kv_cache_dtype.startswith("fp8") else "bf16",
        "new_tokens": new_tokens,
        "timed_steps": steps,
        "layers": shape.layers,
        "prompt_len": {"median": float(prompt.median()), "mean": round(float(prompt.float().mean()), 1),
                       "min": int(prompt.min()), "max": int(prompt.max()),
                       "distribution": f"lognormal(median {median}, sigma {sigma}) clipped [{lo}, {hi}]"},
        "kv_tokens_at_end": int(final_lens.sum().item()),
        "weight_bytes": model.weight_bytes(),
        "logits_finite": finite,
        "data": "synthetic (random-init weights, random prompt K/V, greedy tokens)",
    }


def _run_eager(model: DecoderModel, state: DecodeState, batch: int, new_tokens: int,
               shape: DecoderShape, prompt: torch.Tensor, stream: torch.cuda.Stream,
               kv_cache_dtype: str, dist: tuple) -> dict:
    """Eager steps: the host launches every kernel of every layer, every step."""
    import time

    def step():
        return model.step(state.tokens, state.positions, state.kv_caches, state.meta)

    with torch.cuda.stream(stream):
        logits = step()  # warm-up: the first decoded token (workspace sized here)
        state.tokens.copy_(logits.argmax(-1))
    torch.cuda.synchronize()
    steps = new_tokens - 1
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        t0 = time.perf_counter()
        start.record(stream)
        for _ in range(steps):
            advance(state)
            logits = step()
            state.tokens.copy_(logits.argmax(-1))
        end.record(stream)
        host_s = time.perf_counter() - t0
    torch.cuda.synchronize()
    step_ms = start.elapsed_time(end) / steps

    # Attention alone, eager: the same two backend calls per layer, launched
    # from Python; GPU time from events, host time per layer from the clock.
    q_static = torch.randn(batch, shape.q_heads, shape.head_dim, device=model.device,
                           dtype=model.dtype)
    kv_static = torch.randn(batch, shape.kv_heads, shape.head_dim, device=model.device,
                            dtype=model.dtype)
    attn_static = torch.empty(batch, shape.q_heads * shape.head_dim, device=model.device,
                              dtype=model.dtype)
    reps = 20

    def attention_layers():
        for i in range(shape.layers):
            model.attention(i, q_static, kv_static, kv_static, state.kv_caches[i], state.meta,
                            attn_static)

    a0 = torch.cuda.Event(enable_timing=True)
    a1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        attention_layers()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        a0.record(stream)
        for _ in range(reps):
            attention_layers()
        a1.record(stream)
        attn_host_s = time.perf_counter() - t0
    torch.cuda.synchronize()
    attn_ms = a0.elapsed_time(a1) / reps
    final_lens = state.meta.seq_lens.to(torch.int64)
    kv_bytes_step = (int(final_lens.sum().item()) * shape.kv_heads * shape.head_dim * 2
                     * state.kv_caches[0].element_size() * shape.layers)
    median, sigma, lo, hi = dist
    return {
        "mode": "eager",
        "decode_tok_s": round(batch / (step_ms * 1e-3), 1),
        "step_ms": round(step_ms, 4),
        "host_ms_per_step": round(host_s * 1e3 / steps, 4),
        "attention_ms": round(attn_ms, 4),
        "attention_share": round(attn_ms / step_ms, 4),
        "attention_host_us_per_layer": round(attn_host_s * 1e6 / (reps * shape.layers), 2),
        "attention_kv_gb_s": round(kv_bytes_step / (attn_ms * 1e-3) / 1e9, 1),
        "batch": batch,
        "kv_cache_dtype": "fp8_e4m3" if kv_cache_dtype.startswith("fp8") else "bf16",
        "new_tokens": new_tokens,
        "timed_steps": steps,
        "layers": shape.layers,
        "prompt_len": {"median": float(prompt.median()),
                       "mean": round(float(prompt.float().mean()), 1),
                       "min": int(prompt.min()), "max": int(prompt.max()),
                       "distribution": f"lognormal(median {median}, sigma {sigma}) clipped "
                                       f"[{lo}, {hi}]"},
        "kv_tokens_at_end": int(final_lens.sum().item()),
        "logits_finite": bool(torch.isfinite(logits.float()).all().item()),
        "data": "synthetic (random-init weights, random prompt K/V, greedy tokens)",
    }


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--batch", type=int, default=128)
    ap.add_argument("--new-tokens", type=int, default=256)
    ap.add_argument("--layers", type=int, default=QWEN3_4B.layers)
    ap.add_argument("--kv-cache-dtype", default="auto", choices=("auto", "fp8"))
    ap.add_argument("--eager", action="store_true",
                    help="launch every step from Python instead of replaying a HIP graph")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("decode_step needs a GPU", file=sys.stderr)
        return 2
    shape = DecoderShape(layers=args.layers)
    print(json.dumps(run(args.batch, args.new_tokens, shape,
                         kv_cache_dtype=args.kv_cache_dtype, eager=args.eager)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
