"""Every kernel launch that bench.py times, at the shape and through the entry point it is timed
with, against the oracle.

* The headline step's int4 linears at M = 1 (symmetric codes, fp32 group scales) through
  ``sqx_int4_linear`` with the library's launch shape: the fused gate/up projection 4096 -> 28672
  (more than 1024 tiles, one round per wave: the 8-wave-per-SIMD one-row form) and the lm_head
  4096 -> 128256 (8016 tiles, sampled rows).
* BASELINE config 2's own format (uint4 codes with bf16 scale and zero per group) at the four
  Llama-3-8B shapes and M in {1, 4, 8}, through ``sqx_int4_linear`` as the bench calls it and through
  ``int4_linear_tiled``.
* Config 4's MXFP4 weights x bf16 activations at M = 4096 on both Llama-3-70B MLP shapes (the prefill
  row), sampled rows and columns.
* Config 5's decode step at full width: the 32-layer Llama-3-8B-shaped model's captured step equals
  its eager step bit for bit over two steps at B = 1 and 8, and a two-layer model of the same
  width (context 2048, 2046 cached keys per row, vocab 128256) against the decode oracle on sampled
  logits.

Bars as in the per-format tests: linears within max-abs-rel 1e-2 of the float64 product of the
reference's bf16-cast dequantized weight plus the elementwise bound 2**-7 (|y| + rms y); quantized
codes bit-exact on sampled rows; the decode step within 2x the reference bf16 composition's own
distance to the fp32 run (plus 2**-9 of the logit range).
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from oracle import decode_ref as D
from oracle import quant_ref as R
from tests.conftest import print_case
from tests.test_gpu_int4 import _check_linear

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def mods():
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import int4_group, nvfp4_mxfp4

    return _lib, _lib.load(), int4_group, nvfp4_mxfp4


def _s():
    return torch.cuda.current_stream().cuda_stream


def _sample_rows(n: int, count: int, seed: int) -> np.ndarray:
    if count >= n:
        return np.arange(n)
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([np.arange(16), np.arange(n - 16, n), rng.choice(n, count, replace=False)]))


@pytest.mark.parametrize("n,k,rows", [(28672, 4096, 28672), (128256, 4096, 8192)], ids=["gate_up", "lm_head"])
def test_headline_one_row_linear(mods, n, k, rows):
    """The dominant launch of the headline step (gate/up) and the lm_head, M = 1, as bench.py issues
    them: ``sqx_int4_linear`` with k_slices = 0 (the library's launch shape)."""
    _lib, lib, i4, _ = mods
    print_case("headline one-row linear", n, k)
    g = torch.Generator(device=DEV).manual_seed(1000 + n)
    w = (torch.randn(n, k, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    q, s = i4.quantize_groupwise_int4(w)
    tw = i4.tile_int4(q, s)
    x = torch.randn(1, k, device=DEV, generator=g).to(torch.bfloat16)
    y = torch.empty(1, n, dtype=torch.bfloat16, device=DEV)
    rc = lib.sqx_int4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32, x.data_ptr(), _lib.DTYPE_BF16,
                             y.data_ptr(), None, 1, n, k, 128, 0, _s())
    assert rc == 0, lib.sqx_last_error().decode()
    torch.cuda.synchronize()
    ri = _sample_rows(n, rows, n)
    rit = torch.from_numpy(ri).to(DEV)
    qn, sn = q[rit].cpu().numpy(), s[rit].cpu().numpy()
    qr, sr = R.quantize_groupwise_int4(w[rit[:64]].float().cpu().numpy())  # the codes themselves, bit-exact
    assert np.array_equal(qn[:64], qr) and np.array_equal(sn[:64].view(np.uint32), sr.view(np.uint32))
    w_eff = R.round_bf16(R.dequantize_groupwise_int4(qn, sn))
    _check_linear(y[:, rit], R.linear_f64(x.float().cpu().numpy(), w_eff), f"one-row {k}->{n}")
    # the functional API takes the same launch and gives the same bits
    assert torch.equal(y, i4.int4_linear_tiled(x, tw))


@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)],
                         ids=lambda v: str(v))
def test_config2_asymmetric_bf16_params(mods, n, k):
    """uint4 codes, bf16 scale and zero per group of 128, M in {1, 4, 8}, at every
    Llama-3-8B shape. Codes, scales and zeros bit-exact on sampled rows; the linear through the entry
    point the bench times (``sqx_int4_linear``, k_slices = 0) and through ``int4_linear_tiled``. The
    asymmetric format has no reference symbol: its oracle is pinned by the affine invariants of
    tests/test_oracle_int4.py, not by the reference."""
    _lib, lib, i4, _ = mods
    print_case("config2 asym", n, k)
    g = torch.Generator(device=DEV).manual_seed(1002 + n + k)
    w = torch.randn(n, k, device=DEV, generator=g) * 0.02
    qa, sa, za = i4.quantize_groupwise_uint4_asym(w, 128, torch.bfloat16)
    ri = torch.from_numpy(_sample_rows(n, 48, k)).to(DEV)
    qr, sr, zr = R.quantize_groupwise_uint4_asym(w[ri].cpu().numpy(), 128, param="bf16")
    assert np.array_equal(qa[ri].cpu().numpy(), qr)
    assert np.array_equal(sa[ri].float().cpu().numpy(), sr) and np.array_equal(za[ri].float().cpu().numpy(), zr)
    tw = i4.tile_int4(qa, sa, za, 128)
    qn, sn, zn = qa.cpu().numpy(), sa.float().cpu().numpy(), za.float().cpu().numpy()
    w_eff = R.round_bf16(R.dequantize_groupwise_uint4_asym(qn, sn, zn))
    del w
    for m in (1, 4, 8):
        x = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
        y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        rc = lib.sqx_int4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), tw.zt.data_ptr(), _lib.DTYPE_BF16, x.data_ptr(),
                                 _lib.DTYPE_BF16, y.data_ptr(), None, m, n, k, 128, 0, _s())
        assert rc == 0, lib.sqx_last_error().decode()
        y_ref = R.linear_f64(x.float().cpu().numpy(), w_eff)
        _check_linear(y, y_ref, f"asym {k}->{n} M={m} (sqx_int4_linear)")
        _check_linear(i4.int4_linear_tiled(x, tw), y_ref, f"asym {k}->{n} M={m} (int4_linear_tiled)")


@pytest.mark.parametrize("n,k", [(28672, 8192), (8192, 28672)], ids=["8192to28672", "28672to8192"])
def test_config4_mxfp4_weights_bf16_m4096(mods, n, k):
    """Config 4's MXFP4 weights x bf16 activations at M = 4096 (the prefill row bench.py times through
    ``fp4_linear_tiled``): 24 rows x 160 columns of y against the float64 product of the bf16
    activations and the oracle-dequantized weight rows (every MXFP4 value is exact in bf16), within
    the fp32-accumulation bound plus half a bf16 ulp of the output."""
    _, _, _, f4 = mods
    m = 4096
    print_case("config4 mxfp4 x bf16", m, n, k)
    g = torch.Generator(device=DEV).manual_seed(1004 + n)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    tw = f4.tile_fp4(f4.mxfp4_quantize(w, 32))
    y = f4.fp4_linear_tiled(x, tw)
    torch.cuda.synchronize()
    rng = np.random.default_rng(n)
    ri = np.sort(np.concatenate([[0, m - 1], rng.choice(np.arange(1, m - 1), 22, replace=False)]))
    ci = np.sort(np.concatenate([[0, n - 1], rng.choice(np.arange(1, n - 1), 158, replace=False)]))
    wr = w[torch.from_numpy(ci).to(DEV)].cpu().numpy()
    codes, s_block, _, _, nn_ = R.mxfp4_quantize(wr.reshape(-1), 32)
    wd = R.mxfp4_dequantize(codes, s_block, wr.shape, nn_).astype(np.float64)
    assert np.array_equal(R.round_bf16(wd), wd)
    xs = x[torch.from_numpy(ri).to(DEV)].float().cpu().numpy().astype(np.float64)
    y_ref = xs @ wd.T
    mag = np.abs(xs) @ np.abs(wd).T
    ys = y[torch.from_numpy(ri).to(DEV)][:, torch.from_numpy(ci).to(DEV)].float().cpu().numpy().astype(np.float64)
    err = np.abs(ys - y_ref)
    bound = (k / 32 + 8) * 2.0**-24 * mag + 2.0**-8 * np.abs(y_ref) + 1e-30
    worst = float((err / bound).max())
    assert worst <= 1.0, f"config4 bf16 x {m}x{k}->{n}: {worst:.2f}x the accumulation + rounding bound"
    _check_linear(torch.from_numpy(ys), y_ref, f"config4 bf16 x {m}x{k}->{n}")


# ---------------------------------------------------------------------------------------------- config 5
def _fill_cache(st, seed: int, length: int) -> None:
    g = torch.Generator(device=DEV).manual_seed(seed)
    st.k.normal_(generator=g)
    st.v.normal_(generator=g)
    st.set_lengths([length] * st.batch)


@pytest.mark.parametrize("B", [1, 8])
def test_config5_full_model_graph_equals_eager(B):
    """The 32-layer Llama-3-8B-shaped step (vocab 128256, context 2048, 2047 cached keys per row):
    two captured replays equal two eager steps bit for bit (logits, picks, cache, lengths)."""
    from scratch_llm_amd.decode import LLAMA3_8B, Int4DecodeLM

    print_case("config5 full model graph == eager", B)
    cfg = LLAMA3_8B
    model = Int4DecodeLM.random_init(cfg, DEV, seed=1005)
    ctx = cfg.context_length
    a, b = model.new_state(B, ctx), model.new_state(B, ctx)
    _fill_cache(a, 7 + B, ctx - 1)
    _fill_cache(b, 7 + B, ctx - 1)
    tok = torch.randint(0, cfg.vocab_size, (B,), generator=torch.Generator().manual_seed(B))
    a.set_tokens(tok, cfg.vocab_size)
    b.set_tokens(tok, cfg.vocab_size)
    graph = model.capture(b)
    for t in range(2):
        model.step(a)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(a.logits, b.logits), f"step {t}: logits"
        assert torch.equal(a.tokens, b.tokens), f"step {t}: picks"
        assert torch.equal(a.lengths, b.lengths)
        assert bool(torch.isfinite(a.logits.float()).all())
    assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)
    del graph, a, b, model
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B", [1, 3, 8, 32, 64])
def test_config5_full_width_against_oracle(B):
    """A two-layer model at Llama-3-8B width (d 4096, 32 q / 8 kv heads, SwiGLU 14336, vocab 128256,
    context 2048 with 2046 random cached keys per row) for two steps against the decode oracle's bf16
    composition and fp32 run on 8192 sampled logits; the second layer reads the first's residual sums
    at B = 1. At B = 32 and 64 the step runs every row (the row-tiled linears, K-split partials folded
    into the norms, one attention chunk per row) and the oracle follows 8 sampled rows (rows do not
    interact). Codes of the quantized weights are bit-exact with the oracle quantizer on sampled rows,
    and the oracle dequantizes the same codes."""
    from scratch_llm_amd.decode import LLAMA3_8B, Int4DecodeLM
    from scratch_llm_amd.quant import int4_group as i4

    print_case("config5 full width vs oracle", B)
    cfg = dataclasses.replace(LLAMA3_8B, n_layers=2)
    ctx = cfg.context_length
    gd = torch.Generator(device=DEV).manual_seed(5000 + B)
    hd = cfg.head_dim
    shapes = {"attn.q_proj": (cfg.n_heads * hd, cfg.d_model), "attn.k_proj": (cfg.n_kv_heads * hd, cfg.d_model),
              "attn.v_proj": (cfg.n_kv_heads * hd, cfg.d_model), "attn.o_proj": (cfg.d_model, cfg.n_heads * hd),
              "ffn.w1": (cfg.d_ff, cfg.d_model), "ffn.w3": (cfg.d_ff, cfg.d_model), "ffn.w2": (cfg.d_model, cfg.d_ff)}
    p: dict[str, torch.Tensor] = {"token_emb.weight": torch.randn(cfg.vocab_size, cfg.d_model, device=DEV,
                                                                  generator=gd).to(torch.bfloat16)}
    for i in range(cfg.n_layers):
        for n, shp in shapes.items():
            p[f"blocks.{i}.{n}.weight"] = torch.randn(*shp, device=DEV, generator=gd) * 0.02
        for n in ("attn_norm", "ffn_norm"):
            p[f"blocks.{i}.{n}.weight"] = (1.0 + 0.1 * torch.randn(cfg.d_model, device=DEV, generator=gd)).bfloat16()
    p["final_norm.weight"] = (1.0 + 0.1 * torch.randn(cfg.d_model, device=DEV, generator=gd)).bfloat16()
    p["lm_head.weight"] = torch.randn(cfg.vocab_size, cfg.d_model, device=DEV, generator=gd) * 0.02
    model = Int4DecodeLM.from_state_dict(cfg, lambda n: p[n], DEV)

    cols = _sample_rows(cfg.vocab_size, 8192, 11)
    colt = torch.from_numpy(cols).to(DEV)

    def deq(name: str, rows=None) -> torch.Tensor:
        w = p[name] if rows is None else p[name][rows]
        q, s = i4.quantize_groupwise_int4(w.float())
        rs = torch.arange(0, q.shape[0], max(1, q.shape[0] // 32), device=DEV)[:32]
        qr, sr = R.quantize_groupwise_int4(w[rs].float().cpu().numpy())
        assert np.array_equal(q[rs].cpu().numpy(), qr), f"{name}: codes"
        return torch.from_numpy(R.dequantize_groupwise_int4(q.cpu().numpy(), s.cpu().numpy()))

    ref32 = D.RefModel(cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, hd, ctx, cfg.rope_theta, cfg.norm_eps,
                       embed=p["token_emb.weight"].cpu().float(), final_norm=p["final_norm.weight"].cpu().float())
    for i in range(cfg.n_layers):
        for n in D.LINEAR_NAMES:
            ref32.linears[f"blocks.{i}.{n}"] = deq(f"blocks.{i}.{n}.weight")
        for n in ("attn_norm", "ffn_norm"):
            ref32.norms[f"blocks.{i}.{n}"] = p[f"blocks.{i}.{n}.weight"].cpu().float()
    ref32.linears["lm_head"] = deq("lm_head.weight", colt)
    ref16 = dataclasses.replace(ref32, embed=ref32.embed.bfloat16(), final_norm=ref32.final_norm.bfloat16(),
                                norms={kk: v.bfloat16() for kk, v in ref32.norms.items()})

    st = model.new_state(B, ctx)
    _fill_cache(st, 17 + B, ctx - 2)  # the two steps write positions 2046 and 2047, the last RoPE rows
    if B <= 8:
        rows = list(range(B))
    else:
        rows = sorted({0, B - 1, *np.random.default_rng(B).choice(B, 6, replace=False).tolist()})
    rt = torch.tensor(rows)
    caches = {}
    for dt in (torch.bfloat16, torch.float32):
        c = D.RefCache.empty(ref32, len(rows), ctx, dt)
        for li in range(cfg.n_layers):
            c.k[li].copy_(st.k[li][rt.to(DEV)].cpu().to(dt))
            c.v[li].copy_(st.v[li][rt.to(DEV)].cpu().to(dt))
        c.lengths[:] = ctx - 2
        caches[dt] = c
    tok = torch.randint(0, cfg.vocab_size, (B,), generator=torch.Generator().manual_seed(B + 1))
    for t in range(2):
        print_case("config5 full width step", B, t)
        nxt = model.step(st, tok)
        torch.cuda.synchronize()
        got = st.logits[rt.to(DEV)][:, colt].float().cpu()
        l16 = D.decode_step(ref16, caches[torch.bfloat16], tok[rt], torch.bfloat16).float()
        l32 = D.decode_step(ref32, caches[torch.float32], tok[rt], torch.float32)
        scale = float(l32.abs().max())
        e_hip = float((got - l32).abs().max())
        e_ref = float((l16 - l32).abs().max())
        assert e_hip <= 2 * e_ref + 2.0**-9 * scale, f"B={B} t={t}: |hip-f32| {e_hip:.4g} vs |bf16 ref-f32| {e_ref:.4g}"
        assert torch.equal(nxt.cpu().long(), st.logits.float().argmax(-1).cpu())
        assert st.lengths.cpu().tolist() == [ctx - 1 + t] * B
        assert caches[torch.float32].lengths.tolist() == [ctx - 1 + t] * len(rows)
        tok = nxt.cpu().long()
    del model, st, p
    torch.cuda.empty_cache()
