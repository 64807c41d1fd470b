"""Named synthetic workloads for the decode path (shapes, formats, seeds).

Each is a seeded synthetic Llama model: matrices N(0, 0.02), norms 1.0,
prompts of uniform random token ids from seed + 1.
"""
from __future__ import annotations

from dataclasses import dataclass

from . import GGML_F32, GGML_Q4_0, GGML_Q6_K, GGML_Q8_0, SynthSpec


@dataclass(frozen=True)
class Workload:
    name: str
    spec: SynthSpec
    prompt_len: int
    decode_steps: int


def tiny_f32() -> Workload:
    """dim 288, 6 layers, 6 heads (hd 48), 6 KV heads, FFN 768, vocab 512,
    ctx 256, all F32, seed 42; 8-token prompt + 64 greedy steps."""
    s = SynthSpec(n_layer=6, n_head=6, n_head_kv=6, n_embd=288, n_ff=768, vocab_size=512,
                  context_length=256, rope_freq_base=10000.0, rms_eps=1e-5,
                  layer_type=GGML_F32, output_type=GGML_F32, embd_type=GGML_F32, seed=42,
                  name="tiny_f32")
    return Workload("tiny_f32", s, 8, 64)


def gqa_q8() -> Workload:
    """dim 512, 8 layers, 8 heads (hd 64), 2 KV heads, FFN 1376, vocab 4096,
    ctx 1024, Q8_0 matrices (output too), F32 embedding; 16 + 256 steps."""
    s = SynthSpec(n_layer=8, n_head=8, n_head_kv=2, n_embd=512, n_ff=1376, vocab_size=4096,
                  context_length=1024, layer_type=GGML_Q8_0, output_type=GGML_Q8_0,
                  embd_type=GGML_F32, seed=43, name="gqa_q8")
    return Workload("gqa_q8", s, 16, 256)


def mistral7b_q4(ctx: int = 4096) -> Workload:
    """Mistral-7B shape: dim 4096, 32 layers, 32 heads (hd 128), 8 KV heads,
    FFN 14336, vocab 32000, RoPE theta 1e6; Q4_0 matrices, output.weight
    Q6_K; KV sized to ctx 4096; 32-token prompt + 128 greedy steps."""
    s = SynthSpec(n_layer=32, n_head=32, n_head_kv=8, n_embd=4096, n_ff=14336, vocab_size=32000,
                  context_length=ctx, rope_freq_base=1e6, layer_type=GGML_Q4_0,
                  output_type=GGML_Q6_K, embd_type=GGML_Q4_0, seed=44, name="mistral7b_q4")
    return Workload("mistral7b_q4", s, 32, 128)


def mistral7b_q8_long(prefix: int = 16384, steps: int = 64) -> Workload:
    """Same 7B shape, every matrix Q8_0, KV filled to `prefix` positions then
    `steps` greedy steps (KV capacity prefix + steps)."""
    s = SynthSpec(n_layer=32, n_head=32, n_head_kv=8, n_embd=4096, n_ff=14336, vocab_size=32000,
                  context_length=prefix + steps, rope_freq_base=1e6, layer_type=GGML_Q8_0,
                  output_type=GGML_Q8_0, embd_type=GGML_Q8_0, seed=45, name="mistral7b_q8_long")
    return Workload("mistral7b_q8_long", s, prefix, steps)


def bytes_per_token_weights(spec: SynthSpec) -> int:
    """Weight bytes one decode step streams (all matrices except the
    embedding, of which one row is read, plus the F32 norms)."""
    from . import BLOCK
    def nbytes(rows, cols, t):
        be, bb = BLOCK[t]
        return rows * (cols // be) * bb
    c, ff, kv, V = spec.n_embd, spec.n_ff, spec.kv_dim, spec.vocab_size
    t = spec.layer_type
    per_layer = (nbytes(c, c, t) + 2 * nbytes(kv, c, t) + nbytes(c, c, t) + 2 * nbytes(ff, c, t)
                 + nbytes(c, ff, t) + 2 * c * 4)
    return (spec.n_layer * per_layer + nbytes(V, c, spec.output_type) + c * 4
            + nbytes(1, c, spec.embd_type))


def prefill_flops(spec: SynthSpec, n: int, p0: int = 0) -> tuple:
    """(projection flops, attention flops) of a prompt of n tokens at
    positions p0 .. p0 + n - 1: 2 per weight per token for the layer
    matrices, and 4 * n_head * head_dim per (query, visible position) pair
    for the scores and the weighted sum."""
    c, ff, kv = spec.n_embd, spec.n_ff, spec.kv_dim
    params = spec.n_layer * (2 * c * c + 2 * kv * c + 3 * ff * c)
    pairs = sum(p0 + t + 1 for t in range(n))
    hd = c // spec.n_head
    return 2 * params * n, spec.n_layer * 4 * spec.n_head * hd * pairs


def kv_bytes_per_position(spec: SynthSpec) -> int:
    """K and V bytes per cached position across all layers (f32)."""
    return spec.n_layer * 2 * spec.kv_dim * 4
