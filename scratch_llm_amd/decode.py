"""One decode step of a Llama-shaped model whose linears are INT4-g128, on MI355X.

The reference decodes by calling ``TransformerLM.forward`` (src/scratch_llm/model.py:439-505) with
one token per row against a slot KV cache (kv_cache.py:80-262, dense ``BatchedKVCache`` storage)
and picking the next token greedily (sampling.py:80-83); with the quantized drop-ins every Linear
is ``w4a16_linear`` (int4_group.py:148-164). This module is that step on the library's kernels:

* the INT4 linears on the tiled weights (the streaming decode kernel below 64 rows, the
  dequant-GEMM from 64 rows), with q|k|v fused into one projection and gate|up into another
  (concatenating rows keeps every group scale: groups run along the input dimension);
* everything between them from sqx_decode.hip: residual add + RMSNorm, split-key GQA attention
  with RoPE and the cache write folded in, SiLU-gate, embedding rows, greedy pick, ``advance``.

A step allocates nothing: :class:`DecodeState` holds the cache and every buffer for one batch
size, so :meth:`Int4DecodeLM.capture` can record the whole step in a HIP graph whose replays
decode token after token (the pick of one replay is the input of the next).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch
from torch import Tensor

from scratch_llm_amd import _lib
from scratch_llm_amd.quant import int4_group as i4

__all__ = ["DecodeConfig", "DecodeState", "Int4DecodeLM", "LLAMA3_8B", "rope_tables"]

# Batches of 2..64 rows run the linears through sqx_int4_skinny's shape choice (the GEMV or a
# decode-regime kernel, K split into the state's workspace); larger batches run the prefill GEMM.
_SKINNY_MAX_M = i4.GEMM_MIN_M - 1


@dataclass(frozen=True)
class DecodeConfig:
    """Architecture of the decoded model (the fields of model.py:57-112 that a decode step reads)."""

    vocab_size: int = 128256
    d_model: int = 4096
    n_layers: int = 32
    n_heads: int = 32
    n_kv_heads: int = 8
    d_ff: int = 14336
    context_length: int = 2048
    rope_theta: float = 10000.0
    norm_eps: float = 1e-5
    group_size: int = 128

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    def validate(self) -> None:
        if self.d_model % self.n_heads != 0:
            raise ValueError(f"d_model={self.d_model} not divisible by n_heads={self.n_heads}")
        if self.n_heads % self.n_kv_heads != 0:
            raise ValueError(f"n_heads={self.n_heads} not divisible by n_kv_heads={self.n_kv_heads}")
        if self.head_dim != 128:
            raise ValueError(f"head_dim={self.head_dim}: the decode attention kernel is built for 128")
        if self.n_heads // self.n_kv_heads not in (1, 2, 4, 8):
            raise ValueError(f"{self.n_heads // self.n_kv_heads} query heads per kv head (1, 2, 4 or 8 are built)")
        for name, k in (("d_model", self.d_model), ("d_ff", self.d_ff)):
            if k % self.group_size != 0:
                raise ValueError(f"{name}={k} not divisible by group_size={self.group_size}")


LLAMA3_8B = DecodeConfig()


def rope_tables(head_dim: int, max_seq_len: int, theta: float) -> tuple[Tensor, Tensor]:
    """cos/sin [max_seq_len, head_dim/2] fp32, computed on the host exactly as the reference's
    RotaryPositionalEmbedding buffers are (model.py:196-202, built on the CPU at construction)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    positions = torch.arange(max_seq_len).float()
    freqs = torch.outer(positions, inv_freq)
    return freqs.cos(), freqs.sin()


@dataclass
class _Layer:
    attn_norm: Tensor
    wqkv: i4.Int4Tiled
    wo: i4.Int4Tiled
    ffn_norm: Tensor
    w13: i4.Int4Tiled
    w2: i4.Int4Tiled


class DecodeState:
    """The slot cache and the step's buffers for one batch size (BatchedKVCache, kv_cache.py:234-262).

    ``k``/``v``: ``[n_layers, B, Hkv, max_ctx, hd]``, bf16, or with ``kv_dtype="fp8"`` E4M3 codes (uint8)
    with fp32 per-(layer, kv head) scales ``k_scale``/``v_scale`` ``[n_layers, Hkv]`` (the per-head FP8
    cache of fp8_kv_per_head.py; set them with :meth:`set_kv_scales` before decoding, static after).
    ``lengths`` int32 ``[B]`` (valid positions before the next write); ``active`` uint8 ``[B]`` (rows that
    ``advance`` bumps); ``tokens`` int32 ``[B]``: the step's input ids, overwritten by its greedy picks;
    ``logits`` bf16 ``[B, vocab]``.
    """

    def __init__(self, model: "Int4DecodeLM", batch: int, max_ctx: int, kv_dtype: str = "bf16") -> None:
        cfg, dev = model.cfg, model.device
        if batch < 1 or max_ctx < 1:
            raise ValueError("batch and max_ctx must be >= 1")
        if max_ctx > cfg.context_length:
            raise ValueError(f"max_ctx={max_ctx} exceeds context_length={cfg.context_length}")
        if kv_dtype not in ("bf16", "fp8"):
            raise ValueError(f"kv_dtype must be 'bf16' or 'fp8', got {kv_dtype!r}")
        self.batch, self.max_ctx, self.kv_dtype = batch, max_ctx, kv_dtype
        hkv, hd, d = cfg.n_kv_heads, cfg.head_dim, cfg.d_model
        shape = (cfg.n_layers, batch, hkv, max_ctx, hd)
        kvt = torch.bfloat16 if kv_dtype == "bf16" else torch.uint8
        self.k = torch.zeros(shape, dtype=kvt, device=dev)
        self.v = torch.zeros(shape, dtype=kvt, device=dev)
        self.k_scale = self.v_scale = None
        if kv_dtype == "fp8":
            self.k_scale = torch.ones(cfg.n_layers, hkv, dtype=torch.float32, device=dev)
            self.v_scale = torch.ones(cfg.n_layers, hkv, dtype=torch.float32, device=dev)
        self.lengths = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.active = torch.ones(batch, dtype=torch.uint8, device=dev)
        self.tokens = torch.zeros(batch, dtype=torch.int32, device=dev)
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.x = [torch.empty(batch, d, **bf), torch.empty(batch, d, **bf)]  # residual stream (ping-pong)
        self.h = torch.empty(batch, d, **bf)  # normalised input of the next projection
        self.delta = torch.empty(batch, d, **bf)  # o_proj / w2 output
        # steps without norm launches: sums of squares of the residual stream per 16 columns [batch, d/16],
        # left by the linear that wrote it for the norm in the next linear
        self.nss = -(-d // 16)
        self.ss = torch.empty(batch, self.nss, dtype=torch.float32, device=dev)
        self.qkv = torch.empty(batch, (cfg.n_heads + 2 * hkv) * hd, **bf)
        self.q = torch.empty(batch, cfg.n_heads * hd, **bf)  # rotated q (one-row steps: the qkv epilogue's)
        self.attn = torch.empty(batch, cfg.n_heads * hd, **bf)
        self.gu = torch.empty(batch, 2 * cfg.d_ff, **bf)
        self.act = torch.empty(batch, cfg.d_ff, **bf)
        self.logits = torch.empty(batch, cfg.vocab_size, **bf)
        lib = _lib.load()
        nb = max(int(lib.sqx_attn_workspace_bytes(batch, cfg.n_heads, hkv, max_ctx)),
                 int(lib.sqx_attn_partials_workspace_bytes(batch, cfg.n_heads, max_ctx)))
        self.attn_ws = torch.empty(max(nb // 4, 4), dtype=torch.float32, device=dev)
        nb = int(lib.sqx_argmax_workspace_bytes(batch, cfg.vocab_size))
        self.argmax_ws = torch.empty(max(nb // 4, 4), dtype=torch.float32, device=dev)
        gw = 0
        for tw in model.linears():  # K splits of the decode-regime linears, or the prefill GEMM's
            if 2 <= batch <= _SKINNY_MAX_M:
                gw = max(gw, int(lib.sqx_int4_skinny_workspace_bytes(batch, tw.rows, tw.cols, 0)))
            elif batch > _SKINNY_MAX_M:
                gw = max(gw, int(lib.sqx_gemm_workspace_bytes(batch, tw.rows, tw.cols)))
        self.gemm_ws = torch.empty(max(gw // 4, 4), dtype=torch.float32, device=dev) if gw > 0 else None

    def set_kv_scales(self, layer: int, k_scale: Tensor, v_scale: Tensor) -> None:
        """Install a layer's per-head scales (``(Hkv,)`` or ``(1, Hkv, 1, 1)``, e.g. ``per_head_scale`` of a
        calibration block; fp8_kv_per_head.py:160-173)."""
        if self.kv_dtype != "fp8":
            raise ValueError("per-head scales belong to an fp8 cache")
        for dst, src in ((self.k_scale, k_scale), (self.v_scale, v_scale)):
            if src.numel() != dst.shape[1]:
                raise ValueError(f"scale must have {dst.shape[1]} elements (one per kv head), got {tuple(src.shape)}")
            dst[layer].copy_(src.reshape(-1).to(torch.float32))

    def write_kv(self, layer: int, k: Tensor, v: Tensor, start: int = 0) -> None:
        """Store a block ``[B, Hkv, T, hd]`` of keys and values at positions ``start..start+T`` of every slot
        (a prefill's output): copied for a bf16 cache, quantized with the layer's scales for an fp8 one."""
        t = k.shape[2]
        if k.shape != v.shape or k.shape[0] != self.batch or start < 0 or start + t > self.max_ctx:
            raise ValueError(f"block {tuple(k.shape)} does not fit the cache at {start}")
        if self.kv_dtype == "bf16":
            self.k[layer, :, :, start:start + t].copy_(k)
            self.v[layer, :, :, start:start + t].copy_(v)
            return
        from scratch_llm_amd.quant import fp8_kv_per_head as kv8

        ks = self.k_scale[layer].view(1, -1, 1, 1)
        vs = self.v_scale[layer].view(1, -1, 1, 1)
        self.k[layer, :, :, start:start + t].copy_(kv8.quantize_per_head(k, ks).view(torch.uint8))
        self.v[layer, :, :, start:start + t].copy_(kv8.quantize_per_head(v, vs).view(torch.uint8))

    def set_lengths(self, lengths) -> None:
        """Set every slot's valid length (a host list or tensor), e.g. after filling the cache."""
        t = torch.as_tensor(lengths, dtype=torch.int32)
        if t.shape != (self.batch,) or bool((t < 0).any()) or bool((t > self.max_ctx).any()):
            raise ValueError(f"lengths must be {self.batch} values in [0, {self.max_ctx}]")
        self.lengths.copy_(t)

    def set_tokens(self, tokens, vocab_size: int) -> None:
        t = torch.as_tensor(tokens, dtype=torch.int64)
        if t.shape != (self.batch,):
            raise ValueError(f"expected {self.batch} token ids, got shape {tuple(t.shape)}")
        if t.device.type == "cpu" and (bool((t < 0).any()) or bool((t >= vocab_size).any())):
            raise IndexError(f"token id out of range [0, {vocab_size})")
        self.tokens.copy_(t.to(torch.int32))


class Int4DecodeLM:
    """A TransformerLM (model.py:439-505) with every Linear, the LM head included, in the reference's
    symmetric INT4-g128 format, decoding on one MI355X."""

    def __init__(self, cfg: DecodeConfig, embed: Tensor, layers: list[_Layer], final_norm: Tensor,
                 lm_head: i4.Int4Tiled) -> None:
        cfg.validate()
        self.cfg = cfg
        self.embed = embed
        self.layers = layers
        self.final_norm = final_norm
        self.lm_head = lm_head
        self.device = embed.device
        # Whether the general step's norm runs inside the next linear's prologue: it does not pay (every
        # workgroup of the wide qkv / gate-up / lm_head projections would recompute the whole row's
        # norm), so it stays a kernel of its own unless asked for. SwiGLU's product needs no prologue:
        # the fused gate|up weight's rows alternate in groups of 8, so the fused step forms silu(g) * u
        # in the gate/up epilogue and the general step runs the SiLU kernel of that layout.
        self.fuse_norm = False
        # One-row steps: the o and down projections end in the residual add and leave the sums of
        # squares per 16 columns and bf16(h * gain) of the next norm; the next projection (qkv, gate/up,
        # the lm_head) multiplies its product by the norm's row factor formed from the sums, so no norm
        # after layer 0's costs a launch.
        self.fuse_norm_sums = True
        # Batched steps: when the o / down projection splits K, its fp32 partials go straight to the
        # next residual add + RMSNorm, which adds them in the linear's own order (no reduce launch).
        self.fuse_split_norm = True
        # Batched steps: when the q|k|v projection splits K, the attention kernel adds its fp32 partials
        # (in the projection's own order) as it loads q and the new key and value (no reduce launch).
        self.fuse_qkv_parts = True
        # One-row steps, when set: attention leaves its key-chunk partials (at most 8 per head) and the
        # o projection merges them while it loads its activations (no combine launch). Off: every
        # o-projection workgroup merges every head, which cost more than the launch it saves.
        self.fuse_attn_merge = False
        cos, sin = rope_tables(cfg.head_dim, cfg.context_length, cfg.rope_theta)
        self.cos = cos.to(self.device)
        self.sin = sin.to(self.device)

    # ------------------------------------------------------------------ construction
    @classmethod
    def from_state_dict(cls, cfg: DecodeConfig, get: Callable[[str], Tensor], device: torch.device | str) -> "Int4DecodeLM":
        """Quantize a float model given by its reference parameter names (``token_emb.weight``,
        ``blocks.{i}.attn.{q,k,v,o}_proj.weight``, ``blocks.{i}.ffn.{w1,w2,w3}.weight``,
        ``blocks.{i}.{attn,ffn}_norm.weight``, ``final_norm.weight``, ``lm_head.weight``; model.py:
        125-133, 148-156, 227-253, 372-392, 439-452). ``get(name)`` returns the tensor; each weight
        is quantized on the device with quantize_groupwise_int4 (bit-exact with int4_group.py:108-129)."""
        cfg.validate()
        dev = torch.device(device)
        g = cfg.group_size

        def qw(*names: str, pairs8: bool = False) -> i4.Int4Tiled:
            qs = [i4.quantize_groupwise_int4(get(n).to(dev, torch.float32), g) for n in names]
            if pairs8:  # gate and up rows alternate in groups of 8: tile t holds gate 8t.. then up 8t..
                (q1, s1), (q3, s3) = qs
                q = torch.stack([q1.view(-1, 8, q1.shape[1]), q3.view(-1, 8, q3.shape[1])], 1).reshape(-1, q1.shape[1])
                s = torch.stack([s1.view(-1, 8, s1.shape[1]), s3.view(-1, 8, s3.shape[1])], 1).reshape(-1, s1.shape[1])
            else:
                q = torch.cat([a for a, _ in qs]) if len(qs) > 1 else qs[0][0]
                s = torch.cat([b for _, b in qs]) if len(qs) > 1 else qs[0][1]
            return i4.tile_int4(q.contiguous(), s.contiguous(), None, g)

        def vec(name: str) -> Tensor:
            return get(name).to(dev, torch.bfloat16).contiguous()

        layers = []
        for i in range(cfg.n_layers):
            p = f"blocks.{i}."
            layers.append(_Layer(
                attn_norm=vec(p + "attn_norm.weight"),
                wqkv=qw(p + "attn.q_proj.weight", p + "attn.k_proj.weight", p + "attn.v_proj.weight"),
                wo=qw(p + "attn.o_proj.weight"),
                ffn_norm=vec(p + "ffn_norm.weight"),
                w13=qw(p + "ffn.w1.weight", p + "ffn.w3.weight", pairs8=True),
                w2=qw(p + "ffn.w2.weight"),
            ))
        embed = get("token_emb.weight").to(dev, torch.bfloat16).contiguous()
        return cls(cfg, embed, layers, vec("final_norm.weight"), qw("lm_head.weight"))

    @classmethod
    def random_init(cls, cfg: DecodeConfig, device: torch.device | str, seed: int = 0, std: float = 0.02) -> "Int4DecodeLM":
        """Synthetic weights of the configured shape: linears ~N(0, std) in fp32, generated and
        quantized one at a time on the device; embedding ~N(0, 1); norm gains 1 (model.py:153)."""
        dev = torch.device(device)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        hd = cfg.head_dim
        shapes = {
            "attn.q_proj.weight": (cfg.n_heads * hd, cfg.d_model),
            "attn.k_proj.weight": (cfg.n_kv_heads * hd, cfg.d_model),
            "attn.v_proj.weight": (cfg.n_kv_heads * hd, cfg.d_model),
            "attn.o_proj.weight": (cfg.d_model, cfg.n_heads * hd),
            "ffn.w1.weight": (cfg.d_ff, cfg.d_model),
            "ffn.w3.weight": (cfg.d_ff, cfg.d_model),
            "ffn.w2.weight": (cfg.d_model, cfg.d_ff),
        }

        def get(name: str) -> Tensor:
            if name.endswith("norm.weight"):
                return torch.ones(cfg.d_model, device=dev)
            if name == "token_emb.weight":
                return torch.randn(cfg.vocab_size, cfg.d_model, device=dev, generator=gen)
            if name == "lm_head.weight":
                return torch.randn(cfg.vocab_size, cfg.d_model, device=dev, generator=gen) * std
            return torch.randn(shapes[name.split(".", 2)[2]], device=dev, generator=gen) * std

        return cls.from_state_dict(cfg, get, dev)

    # ------------------------------------------------------------------ queries
    def linears(self) -> list[i4.Int4Tiled]:
        out = []
        for ly in self.layers:
            out += [ly.wqkv, ly.wo, ly.w13, ly.w2]
        return out + [self.lm_head]

    def weight_bytes(self) -> int:
        """HBM bytes one step streams for weights (tiled codes, scales, norm gains)."""
        return sum(tw.nbytes for tw in self.linears()) + sum(
            ly.attn_norm.numel() * 2 + ly.ffn_norm.numel() * 2 for ly in self.layers
        ) + self.final_norm.numel() * 2

    def new_state(self, batch: int, max_ctx: int | None = None, kv_dtype: str = "bf16") -> DecodeState:
        return DecodeState(self, batch, self.cfg.context_length if max_ctx is None else max_ctx, kv_dtype)

    # ------------------------------------------------------------------ the step
    def _linear(self, st: DecodeState, tw: i4.Int4Tiled, x: Tensor, y: Tensor, stream: int) -> None:
        lib = _lib.load()
        m = st.batch
        if 2 <= m <= _SKINNY_MAX_M:  # the library picks the GEMV or a decode-regime kernel by shape
            rc = lib.sqx_int4_skinny(
                tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32, x.data_ptr(), _lib.DTYPE_BF16,
                y.data_ptr(), None, m, tw.rows, tw.cols, tw.group_size, -1, 0, 0, 0, *_lib.ws_args(st.gemm_ws),
                stream,
            )
        elif m > _SKINNY_MAX_M:
            rc = lib.sqx_int4_gemm(
                tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32, x.data_ptr(), _lib.DTYPE_BF16,
                y.data_ptr(), None, m, tw.rows, tw.cols, tw.group_size, *_lib.ws_args(st.gemm_ws), stream,
            )
        else:
            rc = lib.sqx_int4_linear(
                tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32, x.data_ptr(), _lib.DTYPE_BF16,
                y.data_ptr(), None, m, tw.rows, tw.cols, tw.group_size, 0, stream,
            )
        _lib.check(rc, "int4 linear")

    def _delta_linear(self, st: DecodeState, tw: i4.Int4Tiled, x: Tensor, stream: int) -> tuple[int, int]:
        """A linear whose output is the residual delta: ``(pointer, 0)`` to the bf16 delta, or
        ``(workspace, S)`` when its launch splits K into S fp32 partials left for the norm to add."""
        lib, B = _lib.load(), st.batch
        if self.fuse_split_norm and 2 <= B <= _SKINNY_MAX_M:
            S = lib.sqx_int4_skinny_default_splits(B, tw.rows, tw.cols)
            if S >= 2:
                _lib.check(lib.sqx_int4_skinny_partials(
                    tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32, x.data_ptr(), _lib.DTYPE_BF16, B,
                    tw.rows, tw.cols, tw.group_size, *_lib.ws_args(st.gemm_ws), stream), "int4 linear (partials)")
                return st.gemm_ws.data_ptr(), S
        self._linear(st, tw, x, st.delta, stream)
        return st.delta.data_ptr(), 0

    def _norm_linear(self, st: DecodeState, cur: int, delta: int | None, gain: Tensor, tw: i4.Int4Tiled, y: Tensor,
                     stream: int, splits: int = 0, swiglu: bool = False, parts: bool = False) -> int:
        """RMSNorm of the residual stream (after adding ``delta`` when given: a bf16 row, or with
        ``splits`` >= 2 the fp32 partials of a K-split linear) feeding ``tw``; returns the index of the
        buffer that holds the residual stream afterwards. Small batches run it as one kernel when
        ``fuse_norm`` is set (the norm computed in the linear's LDS copy of the activations), otherwise
        as two. ``swiglu``: ``tw`` is the fused gate|up weight and ``y`` [B, d_ff] receives
        bf16(silu(g) * u), formed in the linear's epilogue up to 64 rows. ``parts``: the linear splits K
        and leaves its fp32 partials in ``st.gemm_ws`` for the next kernel to add (``y`` unused)."""
        cfg, lib, B, d = self.cfg, _lib.load(), st.batch, self.cfg.d_model
        nxt = cur if delta is None else 1 - cur
        h_out = None if delta is None else st.x[nxt].data_ptr()
        lin_out = st.gu if swiglu else y
        if self.fuse_norm and splits < 2 and not parts and lib.sqx_int4_prologue_fits(B, d):
            _lib.check(lib.sqx_int4_linear_rmsnorm(
                tw.wt.data_ptr(), tw.st.data_ptr(), st.x[cur].data_ptr(), delta, gain.data_ptr(), cfg.norm_eps, h_out,
                lin_out.data_ptr(), B, tw.rows, tw.cols, tw.group_size, 0, stream), "rmsnorm + int4 linear")
        else:
            if splits >= 2:
                _lib.check(lib.sqx_rmsnorm_partials(st.x[cur].data_ptr(), delta, splits, gain.data_ptr(), cfg.norm_eps,
                                                    B, d, h_out, st.h.data_ptr(), stream), "rmsnorm (partials)")
            else:
                _lib.check(lib.sqx_rmsnorm(st.x[cur].data_ptr(), delta, gain.data_ptr(), cfg.norm_eps, B, d, h_out,
                                           st.h.data_ptr(), stream), "rmsnorm")
            if swiglu and B <= _SKINNY_MAX_M:
                _lib.check(lib.sqx_int4_linear_swiglu(tw.wt.data_ptr(), tw.st.data_ptr(), st.h.data_ptr(), y.data_ptr(),
                                                      B, tw.rows, tw.cols, tw.group_size, stream), "gate|up + silu * up")
                return nxt
            if parts:
                _lib.check(lib.sqx_int4_skinny_partials(
                    tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32, st.h.data_ptr(), _lib.DTYPE_BF16, B,
                    tw.rows, tw.cols, tw.group_size, *_lib.ws_args(st.gemm_ws), stream), "int4 linear (partials)")
                return nxt
            self._linear(st, tw, st.h, lin_out, stream)
        if swiglu:
            _lib.check(lib.sqx_silu_mul_pairs8(st.gu.data_ptr(), B, cfg.d_ff, y.data_ptr(), stream), "silu_mul")
        return nxt

    def _norm_sums_linear(self, st: DecodeState, tw: i4.Int4Tiled, y: Tensor, stream: int) -> None:
        """``tw`` applied to RMSNorm(h) as ``r * (bf16(h * gain) @ W^T)`` per row: ``st.h`` holds
        bf16(h * gain) and ``st.ss`` the sums of squares of h, both left by the residual epilogue of
        the linear that wrote h; the row factor r is formed from the sums in the linear's epilogue."""
        lib = _lib.load()
        _lib.check(lib.sqx_int4_linear_rowscale_sumsq(
            tw.wt.data_ptr(), tw.st.data_ptr(), st.h.data_ptr(), st.ss.data_ptr(), st.nss, self.cfg.norm_eps,
            y.data_ptr(), st.batch, tw.rows, tw.cols, tw.group_size, 0, stream), "rmsnorm (row factor) + int4 linear")

    def _norm_sums_swiglu(self, st: DecodeState, tw: i4.Int4Tiled, y: Tensor, stream: int) -> None:
        """:meth:`_norm_sums_linear` for the fused gate|up weight (gate and up rows alternating in groups
        of 8) with SwiGLU's product in the epilogue: ``y`` [B, d_ff] = bf16(silu(g) * u)."""
        lib = _lib.load()
        _lib.check(lib.sqx_int4_linear_rowscale_swiglu(
            tw.wt.data_ptr(), tw.st.data_ptr(), st.h.data_ptr(), st.ss.data_ptr(), st.nss, self.cfg.norm_eps,
            y.data_ptr(), st.batch, tw.rows, tw.cols, tw.group_size, 0, stream),
            "rmsnorm (row factor) + gate|up + silu * up")

    STEP_KINDS = ("qkv", "attention", "o", "gate_up", "down", "lm_head", "other")

    def step(self, st: DecodeState, tokens=None, only: str | None = None) -> Tensor:
        """Decode one token per row: logits of ``st.tokens`` (or ``tokens``) at each row's position,
        written to ``st.logits``; the greedy picks replace ``st.tokens``; active rows advance. Returns
        ``st.tokens``. Only device work is issued (no host synchronisation).

        ``only`` (one of ``STEP_KINDS``) issues just the launches of that kind, with the arguments the
        full step gives them, for timing each kind's share of the step; the results are then
        meaningless. A norm that runs as a kernel of its own before a linear counts with the linear."""
        cfg, lib = self.cfg, _lib.load()
        if only is not None and only not in self.STEP_KINDS:
            raise ValueError(f"only must be one of {self.STEP_KINDS}, got {only!r}")
        if tokens is not None:
            st.set_tokens(tokens, cfg.vocab_size)
        _lib.require_device(st.tokens, self.embed, fn="Int4DecodeLM.step")
        B, d, H, Hkv, hd, T = st.batch, cfg.d_model, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, st.max_ctx
        s = _lib.stream_ptr(self.device)
        ck = _lib.check

        def go(kind: str) -> bool:
            return only is None or only == kind

        # no norm launches: each residual add ends a linear and leaves the sums of squares its norm needs,
        # and the linear after the norm applies the row factor (one row: the one-row GEMV; 2..8 rows:
        # the multi-row GEMV, where it takes every linear of the step)
        qkv_rows = (H + 2 * Hkv) * hd
        if B == 1:
            sums = (self.fuse_norm_sums and d <= 8192 and lib.sqx_int4_prologue_fits(1, d)
                    and lib.sqx_int4_prologue_fits(1, cfg.d_ff))
        else:
            rf = lib.sqx_int4_rows_fits
            sums = (self.fuse_norm_sums and d <= 8192 and d % 64 == 0 and rf(B, qkv_rows, d, 1) and rf(B, d, d, 0)
                    and rf(B, 2 * cfg.d_ff, d, 1) and rf(B, d, cfg.d_ff, 0) and rf(B, cfg.vocab_size, d, 1))
        # with a bf16 cache: RoPE and the cache write run in the q|k|v projection's epilogue (the one-row
        # form takes fewer than 1024 row tiles of 16; wider projections keep the separate RoPE)
        rope_in_qkv = sums and st.kv_dtype == "bf16" and (B > 1 or qkv_rows // 16 < 1024)
        # one row: the attention combine runs in the o projection's activation load (two 128-column
        # k-blocks per wave)
        kb_o = d // 128
        merge = (self.fuse_attn_merge and sums and B == 1 and d % 256 == 0 and kb_o // 2 <= 16 and H * hd == d)
        # a K-split q|k|v projection (the general step, B >= 48 at Llama-3-8B shapes) leaves its fp32
        # partials and the attention kernel adds them as the projection's reduce would (no reduce launch)
        qkv_split = 0
        if not sums and self.fuse_qkv_parts and 2 <= B <= _SKINNY_MAX_M:
            S = lib.sqx_int4_skinny_default_splits(B, qkv_rows, d)
            qkv_split = S if S >= 2 else 0
        with torch.cuda.device(self.device):
            if go("other"):
                ck(lib.sqx_embed(self.embed.data_ptr(), cfg.vocab_size, st.tokens.data_ptr(), B, d,
                                 st.x[0].data_ptr(), s), "embed")
            cur, delta, dsplit, have_ss = 0, None, 0, False
            for li, ly in enumerate(self.layers):
                # ---- q|k|v (with the attention norm)
                if rope_in_qkv:
                    if not have_ss and go("qkv"):  # layer 0: the norm of the embedding row on its own
                        ck(lib.sqx_rmsnorm(st.x[cur].data_ptr(), None, ly.attn_norm.data_ptr(), cfg.norm_eps, B, d,
                                           None, st.h.data_ptr(), s), "rmsnorm")
                    if go("qkv"):
                        ck(lib.sqx_int4_linear_rope_kv(
                            ly.wqkv.wt.data_ptr(), ly.wqkv.st.data_ptr(), st.h.data_ptr(),
                            st.ss.data_ptr() if have_ss else None, st.nss, cfg.norm_eps,
                            st.lengths.data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(), cfg.context_length, H,
                            Hkv, T, st.q.data_ptr(), st.k[li].data_ptr(), st.v[li].data_ptr(), B, ly.wqkv.rows,
                            ly.wqkv.cols, ly.wqkv.group_size, 0, s), "qkv + rope + cache write")
                elif have_ss:
                    if go("qkv"):
                        self._norm_sums_linear(st, ly.wqkv, st.qkv, s)
                elif go("qkv"):
                    cur = self._norm_linear(st, cur, delta, ly.attn_norm, ly.wqkv, st.qkv, s, dsplit,
                                            parts=qkv_split > 0)
                else:  # the residual stream advances as the norm's launch would have left it
                    cur = cur if delta is None else 1 - cur
                # ---- attention over the cache
                if not go("attention"):
                    pass
                elif merge:  # the partials only; the o projection merges them
                    fp8 = st.kv_dtype == "fp8"
                    ck(lib.sqx_decode_attention_partials(
                        st.q.data_ptr() if rope_in_qkv else st.qkv.data_ptr(), st.lengths.data_ptr(),
                        None if rope_in_qkv else self.cos.data_ptr(), None if rope_in_qkv else self.sin.data_ptr(),
                        cfg.context_length, st.k[li].data_ptr(), st.v[li].data_ptr(),
                        st.k_scale[li].data_ptr() if fp8 else None, st.v_scale[li].data_ptr() if fp8 else None,
                        B, H, Hkv, hd, T, st.attn_ws.data_ptr(), st.attn_ws.numel() * 4, s), "attention partials")
                elif rope_in_qkv:
                    ck(lib.sqx_decode_attention(st.q.data_ptr(), st.k[li].data_ptr(), st.v[li].data_ptr(),
                                                st.lengths.data_ptr(), B, H, Hkv, hd, T, st.attn.data_ptr(),
                                                st.attn_ws.data_ptr(), st.attn_ws.numel() * 4, s), "attention")
                elif qkv_split:
                    fp8 = st.kv_dtype == "fp8"
                    ck(lib.sqx_decode_attention_rope_parts(
                        st.gemm_ws.data_ptr(), qkv_split, st.lengths.data_ptr(), self.cos.data_ptr(),
                        self.sin.data_ptr(), cfg.context_length, st.k[li].data_ptr(), st.v[li].data_ptr(),
                        st.k_scale[li].data_ptr() if fp8 else None, st.v_scale[li].data_ptr() if fp8 else None,
                        B, H, Hkv, hd, T, st.attn.data_ptr(), st.attn_ws.data_ptr(), st.attn_ws.numel() * 4, s),
                       "attention (q|k|v partials)")
                elif st.kv_dtype == "fp8":
                    ck(lib.sqx_decode_attention_rope_fp8kv(
                        st.qkv.data_ptr(), st.lengths.data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(),
                        cfg.context_length, st.k[li].data_ptr(), st.v[li].data_ptr(), st.k_scale[li].data_ptr(),
                        st.v_scale[li].data_ptr(), B, H, Hkv, hd, T, st.attn.data_ptr(), st.attn_ws.data_ptr(),
                        st.attn_ws.numel() * 4, s), "attention")
                else:
                    ck(lib.sqx_decode_attention_rope(
                        st.qkv.data_ptr(), st.lengths.data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(),
                        cfg.context_length, st.k[li].data_ptr(), st.v[li].data_ptr(), B, H, Hkv, hd, T,
                        st.attn.data_ptr(), st.attn_ws.data_ptr(), st.attn_ws.numel() * 4, s), "attention")
                if sums:
                    # o and down end in the residual add and leave bf16(h * gain) of the next norm with
                    # the sums of squares of h; the linear after each norm applies its row factor
                    gain_next = self.layers[li + 1].attn_norm if li + 1 < len(self.layers) else self.final_norm
                    if go("o") and merge:
                        ck(lib.sqx_int4_linear_attn_residual(
                            ly.wo.wt.data_ptr(), ly.wo.st.data_ptr(), st.attn_ws.data_ptr(), st.lengths.data_ptr(), T,
                            st.x[cur].data_ptr(), st.x[1 - cur].data_ptr(), st.ss.data_ptr(), ly.ffn_norm.data_ptr(),
                            st.h.data_ptr(), 1, ly.wo.rows, ly.wo.cols, ly.wo.group_size, kb_o // 2, s),
                           "attention merge + o + residual")
                    elif go("o"):
                        ck(lib.sqx_int4_linear_residual(
                            ly.wo.wt.data_ptr(), ly.wo.st.data_ptr(), st.attn.data_ptr(), st.x[cur].data_ptr(),
                            st.x[1 - cur].data_ptr(), st.ss.data_ptr(), ly.ffn_norm.data_ptr(), st.h.data_ptr(), B,
                            ly.wo.rows, ly.wo.cols, ly.wo.group_size, 0, s), "o + residual")
                    cur = 1 - cur
                    if go("gate_up"):
                        self._norm_sums_swiglu(st, ly.w13, st.act, s)
                    if go("down"):
                        ck(lib.sqx_int4_linear_residual(
                            ly.w2.wt.data_ptr(), ly.w2.st.data_ptr(), st.act.data_ptr(), st.x[cur].data_ptr(),
                            st.x[1 - cur].data_ptr(), st.ss.data_ptr(), gain_next.data_ptr(), st.h.data_ptr(), B,
                            ly.w2.rows, ly.w2.cols, ly.w2.group_size, 0, s), "down + residual")
                    cur, have_ss = 1 - cur, True
                    continue
                if go("o"):
                    delta, dsplit = self._delta_linear(st, ly.wo, st.attn, s)
                else:
                    delta, dsplit = self._delta_plan(st, ly.wo)
                if go("gate_up"):
                    cur = self._norm_linear(st, cur, delta, ly.ffn_norm, ly.w13, st.act, s, dsplit, swiglu=True)
                else:
                    cur = cur if delta is None else 1 - cur
                if go("down"):
                    delta, dsplit = self._delta_linear(st, ly.w2, st.act, s)
                else:
                    delta, dsplit = self._delta_plan(st, ly.w2)
            if not go("lm_head"):
                pass
            elif have_ss:  # the last down projection left bf16(h * final gain) and the sums of squares
                self._norm_sums_linear(st, self.lm_head, st.logits, s)
            else:
                self._norm_linear(st, cur, delta, self.final_norm, self.lm_head, st.logits, s, dsplit)
            if go("other"):
                ck(lib.sqx_argmax(st.logits.data_ptr(), B, cfg.vocab_size, st.tokens.data_ptr(),
                                  st.argmax_ws.data_ptr(), st.argmax_ws.numel() * 4, s), "argmax")
                ck(lib.sqx_advance(st.lengths.data_ptr(), st.active.data_ptr(), B, s), "advance")
        return st.tokens

    def _delta_plan(self, st: DecodeState, tw: i4.Int4Tiled) -> tuple[int, int]:
        """What :meth:`_delta_linear` would return for ``tw``, without launching it."""
        lib, B = _lib.load(), st.batch
        if self.fuse_split_norm and 2 <= B <= _SKINNY_MAX_M:
            S = lib.sqx_int4_skinny_default_splits(B, tw.rows, tw.cols)
            if S >= 2:
                return st.gemm_ws.data_ptr(), S
        return st.delta.data_ptr(), 0

    def capture(self, st: DecodeState) -> torch.cuda.CUDAGraph:
        """Record one :meth:`step` on ``st`` in a HIP graph. Each ``replay()`` decodes the next token
        from ``st.tokens`` and the cache as they are at that moment. Capturing runs nothing, so ``st``
        is unchanged."""
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.device(self.device), torch.cuda.graph(g):
            self.step(st)
        return g
