"""scratch_llm's decode step restated with torch on the CPU — TEST INFRASTRUCTURE ONLY.

Restates, for a model whose linears are INT4-g128 drop-ins, src/scratch_llm/model.py's
TransformerLM forward for one token per row against a dense slot cache: Embedding (:136-145),
RMSNorm (:148-162), RoPE (:185-224), the reference attention math (:173-182, :313-349: scores
q k^T / sqrt(d) in the activation dtype, softmax in fp32 cast back, GQA by repeat_interleave),
SwiGLU (:227-237), the pre-norm block (:394-403), the LM head (:439-505); the slot cache of
kv_cache.py:80-262 (write at min(lengths, max_ctx - 1), attend j <= lengths, advance active rows);
and the greedy pick of sampling.py:80-83. Linears are int4_group.py:148-164's composition:
``F.linear(x, W.to(x.dtype))`` with W the fp32 dequantized weight.

``dtype=torch.bfloat16`` is the reference's own bf16 composition; ``dtype=torch.float32`` runs the
same parameters in fp32 (the accuracy yardstick both bf16 paths are measured against).

Pinning (tests/test_oracle_decode.py):
  step vs full forward ...... cached decode logits == full causal recompute
                              (the law of tests/test_kv_cache.py:34-51)
  write / advance ........... named values of tests/test_batched_cache.py:64-107
  rope ...................... score depends only on the offset (tests/test_model.py:79-94);
                              position 0 is the identity; rotation keeps each pair's norm
  attention ................. one visible key returns its value; GQA == MHA on repeated kv heads;
                              float64 brute force of softmax(q k^T / sqrt d) v
  rmsnorm ................... closed form on constant rows
  rows ...................... bit-identical active rows whatever inactive slots hold
                              (tests/test_batched_cache.py:186-213)
  fp8 cache ................. written values are the dequantized codes of the FP8 oracle
                              (oracle/fp8_ref.py, pinned to torch's float8_e4m3fn cast)
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F
from torch import Tensor


@dataclass
class RefModel:
    """Parameters in the reference's layout: ``linears[name]`` fp32 [out, in] (dequantized INT4),
    norm gains and the embedding as stored (bf16 for a bf16 model)."""

    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    context_length: int
    rope_theta: float
    eps: float
    embed: Tensor
    final_norm: Tensor
    linears: dict[str, Tensor] = field(default_factory=dict)
    norms: dict[str, Tensor] = field(default_factory=dict)


@dataclass
class RefCache:
    """BatchedKVCache (kv_cache.py:234-262): k/v per layer [B, Hkv, max_ctx, hd]; lengths, active.

    With ``k_scale``/``v_scale`` (per layer, ``[Hkv]`` fp32) it is the per-head FP8 cache of
    fp8_kv_per_head.py:93-101 in the slot layout: a written key or value is stored as
    ``(saturating_cast(fp32(x) / scale) * scale).to(dtype)``, the dequantized code the attention reads."""

    k: list[Tensor]
    v: list[Tensor]
    lengths: Tensor
    active: Tensor
    k_scale: list[Tensor] | None = None
    v_scale: list[Tensor] | None = None

    @classmethod
    def empty(cls, m: RefModel, batch: int, max_ctx: int, dtype: torch.dtype, k_scale=None, v_scale=None) -> "RefCache":
        shape = (batch, m.n_kv_heads, max_ctx, m.head_dim)
        return cls([torch.zeros(shape, dtype=dtype) for _ in range(m.n_layers)],
                   [torch.zeros(shape, dtype=dtype) for _ in range(m.n_layers)],
                   torch.zeros(batch, dtype=torch.long), torch.ones(batch, dtype=torch.bool), k_scale, v_scale)

    @staticmethod
    def _fp8(x: Tensor, scale: Tensor) -> Tensor:
        s = scale.to(torch.float32).view(1, -1, 1)
        codes = (x.to(torch.float32) / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        return (codes.to(torch.float32) * s).to(x.dtype)

    def write_decode(self, layer: int, k_new: Tensor, v_new: Tensor) -> None:
        """kv_cache.py:194-205 + :259-261: row b lands at min(lengths[b], max_ctx - 1)."""
        pos = self.lengths.clamp(max=self.k[layer].shape[2] - 1)
        rows = torch.arange(self.lengths.shape[0])
        k, v = k_new[:, :, 0], v_new[:, :, 0]
        if self.k_scale is not None:
            k = self._fp8(k, self.k_scale[layer])
            v = self._fp8(v, self.v_scale[layer])
        self.k[layer][rows, :, pos] = k
        self.v[layer][rows, :, pos] = v

    def advance(self) -> None:
        """kv_cache.py:207-213."""
        self.lengths += self.active.long()


def rmsnorm(x: Tensor, w: Tensor, eps: float) -> Tensor:
    """model.py:158-162."""
    x32 = x.float()
    rms = torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (x32 * rms * w.float()).to(x.dtype)


def rope_tables(head_dim: int, max_seq_len: int, theta: float) -> tuple[Tensor, Tensor]:
    """model.py:196-202."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    freqs = torch.outer(torch.arange(max_seq_len).float(), inv_freq)
    return freqs.cos(), freqs.sin()


def rope(x: Tensor, positions: Tensor, cos_t: Tensor, sin_t: Tensor) -> Tensor:
    """model.py:205-224: x (B, H, s, d); positions (s,) shared or (B, s) per row."""
    cos, sin = cos_t[positions], sin_t[positions]
    if positions.dim() == 2:
        cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    else:
        shape = (1,) * (x.dim() - 2) + cos.shape
        cos, sin = cos.view(shape), sin.view(shape)
    xe, xo = x[..., 0::2], x[..., 1::2]
    return torch.stack((xe * cos - xo * sin, xe * sin + xo * cos), dim=-1).flatten(-2).to(x.dtype)


def attention(q: Tensor, k: Tensor, v: Tensor, mask: Tensor | None) -> Tensor:
    """model.py:173-182 (the eager path decode takes): softmax in fp32, cast to q's dtype."""
    scores = q @ k.transpose(-2, -1) / math.sqrt(q.shape[-1])
    if mask is not None:
        scores = scores.masked_fill(~mask, float("-inf"))
    s = scores.float()
    s = s - s.amax(dim=-1, keepdim=True)
    e = s.exp()
    return (e / e.sum(dim=-1, keepdim=True)).to(q.dtype) @ v


def linear(x: Tensor, w: Tensor) -> Tensor:
    """int4_group.py:148-164 with a dequantized fp32 weight."""
    return F.linear(x, w.to(x.dtype))


def _block_attn(m: RefModel, i: int, h: Tensor, positions: Tensor, cache: RefCache | None,
                cos_t: Tensor, sin_t: Tensor) -> Tensor:
    b, s, _ = h.shape
    H, Hkv, hd = m.n_heads, m.n_kv_heads, m.head_dim
    p = f"blocks.{i}.attn."
    q = linear(h, m.linears[p + "q_proj"]).view(b, s, H, hd).transpose(1, 2)
    k = linear(h, m.linears[p + "k_proj"]).view(b, s, Hkv, hd).transpose(1, 2)
    v = linear(h, m.linears[p + "v_proj"]).view(b, s, Hkv, hd).transpose(1, 2)
    q = rope(q, positions, cos_t, sin_t)
    k = rope(k, positions, cos_t, sin_t)
    if cache is not None:  # slot-cache decode (model.py:281-305)
        cache.write_decode(i, k, v)
        k, v = cache.k[i], cache.v[i]
        k_pos = torch.arange(k.shape[2])
        mask = (k_pos.unsqueeze(0) <= cache.lengths.unsqueeze(1))[:, None, None, :]
    else:  # full causal forward
        q_pos = torch.arange(s).unsqueeze(1)
        mask = torch.arange(s).unsqueeze(0) <= q_pos
    if Hkv != H:
        k = k.repeat_interleave(H // Hkv, dim=1)
        v = v.repeat_interleave(H // Hkv, dim=1)
    out = attention(q, k, v, mask).transpose(1, 2).reshape(b, s, H * hd)
    return linear(out, m.linears[p + "o_proj"])


def _ffn(m: RefModel, i: int, h: Tensor) -> Tensor:
    p = f"blocks.{i}.ffn."
    g = linear(h, m.linears[p + "w1"])
    return linear(g * torch.sigmoid(g) * linear(h, m.linears[p + "w3"]), m.linears[p + "w2"])


def _trunk(m: RefModel, ids: Tensor, positions: Tensor, cache: RefCache | None, dtype: torch.dtype) -> Tensor:
    cos_t, sin_t = rope_tables(m.head_dim, m.context_length, m.rope_theta)
    x = m.embed.to(dtype)[ids]
    for i in range(m.n_layers):
        x = x + _block_attn(m, i, rmsnorm(x, m.norms[f"blocks.{i}.attn_norm"].to(dtype), m.eps), positions,
                            cache, cos_t, sin_t)
        x = x + _ffn(m, i, rmsnorm(x, m.norms[f"blocks.{i}.ffn_norm"].to(dtype), m.eps))
    return rmsnorm(x, m.final_norm.to(dtype), m.eps)


@torch.no_grad()
def decode_step(m: RefModel, cache: RefCache, tokens: Tensor, dtype: torch.dtype) -> Tensor:
    """One token per row (TransformerLM.forward with a SlotKVCache, model.py:470-505): returns the
    logits [B, vocab] in ``dtype`` and advances the cache."""
    ids = tokens.long().view(-1, 1)
    logits = linear(_trunk(m, ids, cache.lengths.unsqueeze(1), cache, dtype), m.linears["lm_head"])
    cache.advance()
    return logits[:, -1]


@torch.no_grad()
def full_forward(m: RefModel, ids: Tensor, dtype: torch.dtype) -> Tensor:
    """The uncached causal forward of ids [B, S] (model.py:470-505 with cache=None): logits [B, S, V]."""
    return linear(_trunk(m, ids.long(), torch.arange(ids.shape[1]), None, dtype), m.linears["lm_head"])


def greedy(logits: Tensor) -> Tensor:
    """sampling.py:82-83 per row."""
    return logits.argmax(dim=-1)


LINEAR_NAMES = ("attn.q_proj", "attn.k_proj", "attn.v_proj", "attn.o_proj", "ffn.w1", "ffn.w2", "ffn.w3")


def int4_model(params: dict[str, Tensor], *, n_layers: int, n_heads: int, n_kv_heads: int,
               context_length: int, rope_theta: float = 10000.0, eps: float = 1e-5,
               group_size: int = 128, dtype: torch.dtype = torch.bfloat16) -> RefModel:
    """A RefModel from float parameters under the reference names (``token_emb.weight``,
    ``blocks.{i}.attn.q_proj.weight``, ..., ``lm_head.weight``): every linear goes through the numpy
    restatement of quantize_groupwise_int4 / dequantize_groupwise_int4 (int4_group.py:108-142);
    norm gains and the embedding are stored in ``dtype`` as a ``model.to(dtype)`` would hold them."""
    from oracle import quant_ref as R

    def deq(name: str) -> Tensor:
        q, s = R.quantize_groupwise_int4(params[name].float().numpy(), group_size)
        return torch.from_numpy(R.dequantize_groupwise_int4(q, s, group_size).astype("float32"))

    d = params["token_emb.weight"].shape[1]
    m = RefModel(n_layers, n_heads, n_kv_heads, d // n_heads, context_length, rope_theta, eps,
                 embed=params["token_emb.weight"].to(dtype), final_norm=params["final_norm.weight"].to(dtype))
    for i in range(n_layers):
        for n in LINEAR_NAMES:
            m.linears[f"blocks.{i}.{n}"] = deq(f"blocks.{i}.{n}.weight")
        for n in ("attn_norm", "ffn_norm"):
            m.norms[f"blocks.{i}.{n}"] = params[f"blocks.{i}.{n}.weight"].to(dtype)
    m.linears["lm_head"] = deq("lm_head.weight")
    return m


def random_params(*, vocab: int, d_model: int, n_layers: int, n_heads: int, n_kv_heads: int, d_ff: int,
                  seed: int, std: float = 0.02) -> dict[str, Tensor]:
    """Seeded float parameters under the reference names: linears ~N(0, std), embedding ~N(0, 1),
    norm gains 1 + N(0, 0.1) (non-trivial gains so that the gain multiply is exercised)."""
    g = torch.Generator().manual_seed(seed)
    hd = d_model // n_heads
    p = {"token_emb.weight": torch.randn(vocab, d_model, generator=g)}
    shapes = {"attn.q_proj": (n_heads * hd, d_model), "attn.k_proj": (n_kv_heads * hd, d_model),
              "attn.v_proj": (n_kv_heads * hd, d_model), "attn.o_proj": (d_model, n_heads * hd),
              "ffn.w1": (d_ff, d_model), "ffn.w3": (d_ff, d_model), "ffn.w2": (d_model, d_ff)}
    for i in range(n_layers):
        for n in LINEAR_NAMES:
            p[f"blocks.{i}.{n}.weight"] = torch.randn(*shapes[n], generator=g) * std
        for n in ("attn_norm", "ffn_norm"):
            p[f"blocks.{i}.{n}.weight"] = 1.0 + 0.1 * torch.randn(d_model, generator=g)
    p["final_norm.weight"] = 1.0 + 0.1 * torch.randn(d_model, generator=g)
    p["lm_head.weight"] = torch.randn(vocab, d_model, generator=g) * std
    return p
