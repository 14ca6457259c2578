"""Decode step on the MI355X: each kernel of sqx_decode.hip through the C ABI
against the CPU restatement of the reference op (oracle/decode_ref.py), then the whole step of
scratch_llm_amd.decode against the oracle's bf16 composition and fp32 run of the same INT4 model.

Bars:
  residual add, RoPE, cache write, embedding, argmax, advance: bit-exact (same fp32 operations,
    one rounding to bf16).
  RMSNorm: within one bf16 ulp of the reference formula evaluated on the CPU (the mean's summation
    order and 1/sqrt differ), and bit-exact on at least 99 % of elements.
  attention, SiLU-gate: |err| <= 2**-8 |ref| + 1e-5 max|v| against float64 (one bf16 rounding of
    an fp32 computation).
  decode step: logits no further from the fp32 run than 2x the reference bf16 composition's own
    distance (plus 2**-9 of the logit range), and greedy picks equal to fp32's wherever fp32's
    top-2 margin exceeds 4x the observed error.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import decode_ref as D
from tests.conftest import print_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def lib():
    from scratch_llm_amd import _lib

    return _lib.load()


def _s():
    return torch.cuda.current_stream().cuda_stream


def _ok(lib, rc):
    assert rc == 0, lib.sqx_last_error().decode()


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    a = x.abs().clamp_min(2.0**-126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


# ---------------------------------------------------------------------------------------------
# kernels
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("rows,d", [(1, 4096), (7, 1024), (64, 4096), (3, 8)])
def test_rmsnorm(lib, rows, d):
    print_case("rmsnorm", rows, d)
    g = torch.Generator().manual_seed(rows * 7 + d)
    x = (torch.randn(rows, d, generator=g) * 3).bfloat16()
    dl = torch.randn(rows, d, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(d, generator=g)).bfloat16()
    xd, dd, wd = x.to(DEV), dl.to(DEV), w.to(DEV)
    h, y, y0 = (torch.empty(rows, d, dtype=torch.bfloat16, device=DEV) for _ in range(3))
    _ok(lib, lib.sqx_rmsnorm(xd.data_ptr(), dd.data_ptr(), wd.data_ptr(), 1e-5, rows, d, h.data_ptr(), y.data_ptr(), _s()))
    _ok(lib, lib.sqx_rmsnorm(xd.data_ptr(), None, wd.data_ptr(), 1e-5, rows, d, None, y0.data_ptr(), _s()))
    torch.cuda.synchronize()
    assert torch.equal(h.cpu(), x + dl)  # bf16 + bf16: fp32 sum, one rounding (model.py:402)
    for got, src in ((y.cpu(), x + dl), (y0.cpu(), x)):
        want = D.rmsnorm(src, w, 1e-5)
        diff = (got.float() - want.float()).abs()
        assert bool((diff <= _bf16_ulp(want.float())).all())
        assert float((diff == 0).float().mean()) >= 0.99


@pytest.mark.parametrize("H,Hkv", [(32, 8), (8, 8), (16, 2)])
def test_rope_kv(lib, H, Hkv):
    print_case("rope_kv", H, Hkv)
    hd, T, ctx = 128, 40, 64
    lengths = [3, 0, T - 1, T + 5, 63][: 5]
    B = len(lengths)
    g = torch.Generator().manual_seed(H + Hkv)
    qkv = (torch.randn(B, (H + 2 * Hkv) * hd, generator=g) * 2).bfloat16()
    cos, sin = D.rope_tables(hd, ctx, 10000.0)
    kc = torch.randn(B, Hkv, T, hd, generator=g).bfloat16()
    vc = torch.randn(B, Hkv, T, hd, generator=g).bfloat16()
    kd, vd = kc.to(DEV), vc.to(DEV)
    q = torch.empty(B, H, hd, dtype=torch.bfloat16, device=DEV)
    ln = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    cd, sd = cos.to(DEV), sin.to(DEV)
    _ok(lib, lib.sqx_rope_kv(qkv.to(DEV).data_ptr(), ln.data_ptr(), cd.data_ptr(), sd.data_ptr(), ctx, B, H, Hkv, hd,
                             T, q.data_ptr(), kd.data_ptr(), vd.data_ptr(), _s()))
    torch.cuda.synchronize()
    pos = torch.tensor(lengths).unsqueeze(1)
    qr = D.rope(qkv[:, : H * hd].view(B, 1, H, hd).transpose(1, 2), pos, cos, sin)
    kr = D.rope(qkv[:, H * hd: (H + Hkv) * hd].view(B, 1, Hkv, hd).transpose(1, 2), pos, cos, sin)
    vr = qkv[:, (H + Hkv) * hd:].view(B, 1, Hkv, hd).transpose(1, 2)
    assert torch.equal(q.cpu(), qr[:, :, 0])
    want_k, want_v = kc.clone(), vc.clone()
    cache = D.RefCache([want_k], [want_v], torch.tensor(lengths), torch.ones(B, dtype=torch.bool))
    cache.write_decode(0, kr, vr)
    assert torch.equal(kd.cpu(), want_k)
    assert torch.equal(vd.cpu(), want_v)


def _attn_case(lib, B, H, Hkv, T, lengths, seed):
    hd = 128
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, hd, generator=g) * 2).bfloat16()
    k = (torch.randn(B, Hkv, T, hd, generator=g) * 2).bfloat16()
    v = torch.randn(B, Hkv, T, hd, generator=g).bfloat16()
    ln = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    out = torch.empty(B, H * hd, dtype=torch.bfloat16, device=DEV)
    nb = lib.sqx_attn_workspace_bytes(B, H, Hkv, T)
    ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    _ok(lib, lib.sqx_decode_attention(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ln.data_ptr(), B, H, Hkv, hd, T,
                                      out.data_ptr(), ws.data_ptr(), nb, _s()))
    torch.cuda.synchronize()
    G = H // Hkv
    got = out.cpu().view(B, H, hd).double()
    for b in range(B):
        L = min(max(lengths[b], 0) + 1, T)
        kk = k[b, :, :L].double().repeat_interleave(G, dim=0)
        vv = v[b, :, :L].double().repeat_interleave(G, dim=0)
        s = torch.einsum("hd,htd->ht", q[b].double(), kk) / math.sqrt(hd)
        p = torch.softmax(s, dim=-1)
        want = torch.einsum("ht,htd->hd", p, vv)
        err = (got[b] - want).abs()
        bound = 2.0**-8 * want.abs() + 1e-5 * vv.abs().max()
        assert float((err / bound).max()) <= 1.0, f"row {b} (L={L}): {float((err / bound).max()):.2f}x the bound"


def test_attention_rows_independent_of_batch(lib):
    """A row's output does not depend on the other rows of the batch at a given key-chunk size: B = 2
    and B = 3 (both with 128-key chunks) agree bit for bit on rows 0 and 1. The chunk size is chosen
    from B, so B = 8 (512-key chunks) may differ in the last bits; rows 0 and 1 of B = 2 and B = 8 are
    each within the attention bound of float64. Cache rows past each length, filled with NaN, reach
    none of them."""
    print_case("attention early rows")
    B, H, Hkv, T, hd = 8, 32, 8, 2048, 128
    g = torch.Generator().manual_seed(77)
    q = (torch.randn(B, H, hd, generator=g) * 2).bfloat16().to(DEV)
    k = (torch.randn(B, Hkv, T, hd, generator=g) * 2).bfloat16()
    v = torch.randn(B, Hkv, T, hd, generator=g).bfloat16()
    lengths = [1000, 37, 2047, 5, 640, 63, 64, 1500]
    for b, n in enumerate(lengths):
        k[b, :, n + 1:] = float("nan")
        v[b, :, n + 1:] = float("nan")
    kd, vd = k.to(DEV), v.to(DEV)
    ln = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    outs = {}
    for nb_rows in (2, 3, 8):
        if nb_rows < 8:
            assert lib.sqx_attn_chunk(nb_rows, Hkv, T) == 128
        out = torch.empty(nb_rows, H * hd, dtype=torch.bfloat16, device=DEV)
        nb = lib.sqx_attn_workspace_bytes(nb_rows, H, Hkv, T)
        ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
        _ok(lib, lib.sqx_decode_attention(q.data_ptr(), kd.data_ptr(), vd.data_ptr(), ln.data_ptr(), nb_rows, H, Hkv,
                                          hd, T, out.data_ptr(), ws.data_ptr(), nb, _s()))
        torch.cuda.synchronize()
        outs[nb_rows] = out.cpu()
    assert torch.isfinite(outs[8].float()).all()
    assert torch.equal(outs[2], outs[3][:2])
    G = H // Hkv
    got = outs[8].view(B, H, hd).double()
    got2 = outs[2].view(2, H, hd).double()
    for b in range(B):
        L = lengths[b] + 1
        kk = k[b, :, :L].double().repeat_interleave(G, dim=0)
        vv = v[b, :, :L].double().repeat_interleave(G, dim=0)
        p = torch.softmax(torch.einsum("hd,htd->ht", q[b].cpu().double(), kk) / math.sqrt(hd), dim=-1)
        want = torch.einsum("ht,htd->hd", p, vv)
        bound = 2.0**-8 * want.abs() + 1e-5 * vv.abs().max()
        assert float(((got[b] - want).abs() / bound).max()) <= 1.0, f"row {b}"
        if b < 2:
            # B = 8 takes 512-key chunks, B = 2 128-key chunks: the row's bits may differ between
            # the two, but both stay within the attention bound, so they agree to twice that bound
            assert float(((got2[b] - want).abs() / bound).max()) <= 1.0, f"row {b} at B=2"
            assert float(((got2[b] - got[b]).abs() / (2 * bound)).max()) <= 1.0, f"row {b}: B=2 vs B=8"


@pytest.mark.parametrize("H,Hkv", [(32, 8), (8, 8), (16, 8), (16, 2)])
def test_attention_ragged(lib, H, Hkv):
    print_case("attention", H, Hkv)
    T = 300
    _attn_case(lib, 6, H, Hkv, T, [0, 1, 16, 255, T - 1, T + 7], seed=H * 10 + Hkv)


@pytest.mark.parametrize("B", [1, 8, 64])
def test_attention_config5_context(lib, B):
    """Llama-3-8B heads at the config-5 context: 2048 keys (lengths 2047), plus ragged rows."""
    print_case("attention config5", B)
    T = 2048
    lengths = [T - 1] * B
    if B > 1:
        lengths[1] = 1000
    _attn_case(lib, B, 32, 8, T, lengths, seed=B)


@pytest.mark.parametrize("B,H,Hkv,T,kv8", [(32, 32, 8, 3000, False), (16, 32, 16, 2500, True)])
def test_attention_one_chunk_long_context(lib, B, H, Hkv, T, kv8):
    """With B * Hkv >= 256 each (row, kv head) takes all its keys as one chunk and the partial kernel
    writes the output itself (no combine launch): within the attention bound of float64 at contexts
    past the multi-chunk walks' 1024 keys, bf16 and E4M3 caches, ragged lengths (0, chunk-walk
    boundaries, T - 1, a full slot), with NaN in every cache row past a row's length."""
    from oracle import fp8_ref as F8

    print_case("attention one chunk", B, H, Hkv, T, kv8)
    assert B * Hkv >= 256 and lib.sqx_attn_chunk(B, Hkv, T) >= T
    hd, G = 128, H // Hkv
    g = torch.Generator().manual_seed(B + T)
    lengths = torch.randint(0, T, (B,), generator=g).tolist()
    lengths[:6] = [T - 1, 0, 1023, 1024, 2047, T + 5]
    q = (torch.randn(B, H, hd, generator=g) * 2).bfloat16()
    if kv8:
        k, v = _valid_codes((B, Hkv, T, hd), g), _valid_codes((B, Hkv, T, hd), g)
        ks = torch.rand(Hkv, generator=g) * 0.01 + 0.001
        vs = torch.rand(Hkv, generator=g) * 0.01 + 0.001
    else:
        k = (torch.randn(B, Hkv, T, hd, generator=g) * 2).bfloat16()
        v = torch.randn(B, Hkv, T, hd, generator=g).bfloat16()
    for b, n in enumerate(lengths):  # never read: NaN there would reach the output
        if kv8:
            k[b, :, n + 1:] = 0x7F
            v[b, :, n + 1:] = 0x7F
        else:
            k[b, :, n + 1:] = float("nan")
            v[b, :, n + 1:] = float("nan")
    out = torch.full((B, H * hd), float("nan"), dtype=torch.bfloat16, device=DEV)
    nb = lib.sqx_attn_workspace_bytes(B, H, Hkv, T)
    ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
    ln = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    kd, vd = k.to(DEV), v.to(DEV)
    if kv8:
        ksd, vsd = ks.to(DEV), vs.to(DEV)
        _ok(lib, lib.sqx_decode_attention_fp8kv(q.to(DEV).data_ptr(), kd.data_ptr(), vd.data_ptr(), ksd.data_ptr(),
                                                vsd.data_ptr(), ln.data_ptr(), B, H, Hkv, hd, T, out.data_ptr(),
                                                ws.data_ptr(), nb, _s()))
    else:
        _ok(lib, lib.sqx_decode_attention(q.to(DEV).data_ptr(), kd.data_ptr(), vd.data_ptr(), ln.data_ptr(), B, H, Hkv,
                                          hd, T, out.data_ptr(), ws.data_ptr(), nb, _s()))
    torch.cuda.synchronize()
    got = out.cpu().view(B, H, hd).double()
    assert torch.isfinite(got).all()
    for b in range(B):
        L = min(lengths[b] + 1, T)
        if kv8:
            kk = torch.from_numpy(F8.e4m3_decode(k[b, :, :L].numpy())).double() * ks.double().view(Hkv, 1, 1)
            vv = torch.from_numpy(F8.e4m3_decode(v[b, :, :L].numpy())).double() * vs.double().view(Hkv, 1, 1)
        else:
            kk, vv = k[b, :, :L].double(), v[b, :, :L].double()
        kk, vv = kk.repeat_interleave(G, dim=0), vv.repeat_interleave(G, dim=0)
        p = torch.softmax(torch.einsum("hd,htd->ht", q[b].double(), kk) / math.sqrt(hd), dim=-1)
        want = torch.einsum("ht,htd->hd", p, vv)
        bound = 2.0**-8 * want.abs() + 1e-5 * vv.abs().max()
        assert float(((got[b] - want).abs() / bound).max()) <= 1.0, f"row {b} (L={L})"


@pytest.mark.parametrize("B,H,Hkv,T", [(5, 32, 8, 300), (1, 32, 8, 2048), (3, 16, 16, 64), (64, 32, 8, 2048)])
def test_fused_rope_attention_equals_two_calls(lib, B, H, Hkv, T):
    """sqx_decode_attention_rope == sqx_rope_kv then sqx_decode_attention, bit for bit (output and cache),
    with the new key anywhere in a chunk, at position 0, and at a full slot (lengths >= T)."""
    print_case("fused rope attention", B, H, Hkv, T)
    hd, ctx = 128, max(T + 16, 64)
    g = torch.Generator().manual_seed(B * 1000 + T)
    lengths = torch.randint(0, T, (B,), generator=g)
    lengths[0] = T - 1
    if B > 1:
        lengths[1] = 0
    if B > 2:
        lengths[2] = T + 9  # a full slot: writes row T - 1, attends all T keys, RoPE at position T + 9
    qkv = (torch.randn(B, (H + 2 * Hkv) * hd, generator=g) * 2).bfloat16().to(DEV)
    cache = torch.randn(2, B, Hkv, T, hd, generator=g).bfloat16().to(DEV)
    cos, sin = (t.to(DEV) for t in D.rope_tables(hd, ctx, 10000.0))
    ln = lengths.to(torch.int32).to(DEV)
    nb = lib.sqx_attn_workspace_bytes(B, H, Hkv, T)
    ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
    outs, caches = [], []
    for fused in (False, True):
        kc, vc = cache[0].clone(), cache[1].clone()
        out = torch.empty(B, H * hd, dtype=torch.bfloat16, device=DEV)
        if fused:
            _ok(lib, lib.sqx_decode_attention_rope(qkv.data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx,
                                                   kc.data_ptr(), vc.data_ptr(), B, H, Hkv, hd, T, out.data_ptr(),
                                                   ws.data_ptr(), nb, _s()))
        else:
            q = torch.empty(B, H, hd, dtype=torch.bfloat16, device=DEV)
            _ok(lib, lib.sqx_rope_kv(qkv.data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx, B, H, Hkv, hd, T,
                                     q.data_ptr(), kc.data_ptr(), vc.data_ptr(), _s()))
            _ok(lib, lib.sqx_decode_attention(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), ln.data_ptr(), B, H, Hkv, hd, T,
                                              out.data_ptr(), ws.data_ptr(), nb, _s()))
        torch.cuda.synchronize()
        outs.append(out)
        caches.append((kc, vc))
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])


@pytest.mark.parametrize("B,T,S,kv8", [(5, 300, 2, False), (64, 2048, 2, False), (64, 2048, 2, True),
                                       (9, 500, 3, True), (20, 100, 8, False)])
def test_attention_rope_parts_equals_reduce_then_rope(lib, B, T, S, kv8):
    """sqx_decode_attention_rope_parts == the S partials added in split order in fp32 and rounded to
    bf16 (what sqx_int4_skinny's reduce writes), then sqx_decode_attention_rope[_fp8kv], bit for bit:
    output and every cache byte, with one key chunk per row (B = 64) and several."""
    print_case("rope attention from partials", B, T, S, kv8)
    H, Hkv, hd, ctx = 32, 8, 128, T + 16
    g = torch.Generator().manual_seed(B * 7 + T + S)
    lengths = torch.randint(0, T, (B,), generator=g)
    lengths[0], lengths[1], lengths[2] = T - 1, 0, T + 3
    parts = torch.randn(S, B, (H + 2 * Hkv) * hd, generator=g) * 1.5
    acc = parts[0].clone()
    for s in range(1, S):
        acc += parts[s]
    qkv = acc.bfloat16().to(DEV)
    if kv8:
        cache = (_valid_codes((B, Hkv, T, hd), g), _valid_codes((B, Hkv, T, hd), g))
        ksd = (torch.rand(Hkv, generator=g) * 0.02 + 0.002).to(DEV)
        vsd = (torch.rand(Hkv, generator=g) * 0.02 + 0.002).to(DEV)
    else:
        cache = (torch.randn(B, Hkv, T, hd, generator=g).bfloat16(), torch.randn(B, Hkv, T, hd, generator=g).bfloat16())
    cos, sin = (t.to(DEV) for t in D.rope_tables(hd, ctx, 10000.0))
    ln = lengths.to(torch.int32).to(DEV)
    pd = parts.to(DEV)
    nb = lib.sqx_attn_workspace_bytes(B, H, Hkv, T)
    ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
    outs, caches = [], []
    for from_parts in (True, False):
        kc, vc = cache[0].to(DEV), cache[1].to(DEV)
        out = torch.empty(B, H * hd, dtype=torch.bfloat16, device=DEV)
        if from_parts:
            _ok(lib, lib.sqx_decode_attention_rope_parts(
                pd.data_ptr(), S, ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx, kc.data_ptr(), vc.data_ptr(),
                ksd.data_ptr() if kv8 else None, vsd.data_ptr() if kv8 else None, B, H, Hkv, hd, T, out.data_ptr(),
                ws.data_ptr(), nb, _s()))
        elif kv8:
            _ok(lib, lib.sqx_decode_attention_rope_fp8kv(
                qkv.data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx, kc.data_ptr(), vc.data_ptr(),
                ksd.data_ptr(), vsd.data_ptr(), B, H, Hkv, hd, T, out.data_ptr(), ws.data_ptr(), nb, _s()))
        else:
            _ok(lib, lib.sqx_decode_attention_rope(
                qkv.data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx, kc.data_ptr(), vc.data_ptr(), B, H,
                Hkv, hd, T, out.data_ptr(), ws.data_ptr(), nb, _s()))
        torch.cuda.synchronize()
        outs.append(out.cpu())
        caches.append((kc.cpu(), vc.cpu()))
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    for a, b in zip(caches[0], caches[1]):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_attention_rope_parts_refuses(lib):
    """Split counts outside 1..64 and a missing scale of an E4M3 cache are refused before any launch."""
    print_case("rope attention from partials refuses")
    d = torch.zeros(64, dtype=torch.float32, device=DEV)
    p = d.data_ptr()
    for S, ks, vs in ((0, None, None), (65, None, None), (2, p, None)):
        rc = lib.sqx_decode_attention_rope_parts(p, S, p, p, p, 64, p, p, ks, vs, 1, 32, 8, 128, 64, p, p, 1 << 20, _s())
        assert rc != 0
        assert "sqx_decode_attention_rope_parts" in lib.sqx_last_error().decode()


def _tiled(n, k, group, seed):
    from scratch_llm_amd.quant import int4_group as i4

    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 0.05).to(DEV)
    q, s = i4.quantize_groupwise_int4(w, group)
    return i4.tile_int4(q, s, None, group)


@pytest.mark.parametrize("m,k,group,with_delta", [(1, 4096, 128, True), (3, 4096, 128, False), (7, 4096, 64, True),
                                                  (2, 1056, 32, True), (8, 1024, 128, True)])
def test_linear_rmsnorm_equals_two_calls(lib, m, k, group, with_delta):
    """sqx_int4_linear_rmsnorm == sqx_rmsnorm then sqx_int4_linear, bit for bit (y and the residual)."""
    print_case("linear+rmsnorm", m, k, group, with_delta)
    n = 528
    tw = _tiled(n, k, group, seed=m + k)
    g = torch.Generator().manual_seed(k)
    x = (torch.randn(m, k, generator=g) * 2).bfloat16().to(DEV)
    dl = torch.randn(m, k, generator=g).bfloat16().to(DEV) if with_delta else None
    gain = (1 + 0.1 * torch.randn(k, generator=g)).bfloat16().to(DEV)
    assert lib.sqx_int4_prologue_fits(m, k) == 1
    h1, h2 = (torch.empty(m, k, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    hn = torch.empty(m, k, dtype=torch.bfloat16, device=DEV)
    y1, y2 = (torch.empty(m, n, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    dp = None if dl is None else dl.data_ptr()
    _ok(lib, lib.sqx_rmsnorm(x.data_ptr(), dp, gain.data_ptr(), 1e-5, m, k, h1.data_ptr() if dl is not None else None,
                             hn.data_ptr(), _s()))
    ks = lib.sqx_int4_linear_default_kslices(m, n, k)  # the GEMV the fused kernel runs
    _ok(lib, lib.sqx_int4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), None, 0, hn.data_ptr(), 1, y1.data_ptr(), None, m, n,
                                 k, group, ks, _s()))
    _ok(lib, lib.sqx_int4_linear_rmsnorm(tw.wt.data_ptr(), tw.st.data_ptr(), x.data_ptr(), dp, gain.data_ptr(), 1e-5,
                                         h2.data_ptr() if dl is not None else None, y2.data_ptr(), m, n, k, group, 0, _s()))
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    if dl is not None:
        assert torch.equal(h1, h2)


@pytest.mark.parametrize("m,f,n", [(1, 14336, 4096), (2, 14336, 4096), (3, 14336, 4096), (4, 14336, 4096),
                                   (5, 2048, 1000), (7, 4096, 1024), (2, 1056, 200)])
def test_linear_silu_equals_two_calls(lib, m, f, n):
    """sqx_int4_linear_silu == sqx_silu_mul then the linear, bit for bit: with the library's choice
    (k_slices 0: the multi-row GEMV's slices where the library's linear of those rows is that kernel)
    against sqx_int4_skinny's choice, and with explicit waves (the GEMV's LDS copy) against
    sqx_int4_linear with the same waves."""
    print_case("linear+silu", m, f, n)
    tw = _tiled(n, f, 32 if f == 1056 else 128, seed=f + m)
    group = tw.group_size
    gu = (torch.randn(m, 2 * f, generator=torch.Generator().manual_seed(m)) * 3).bfloat16().to(DEV)
    act = torch.empty(m, f, dtype=torch.bfloat16, device=DEV)
    y1, y2 = (torch.empty(m, n, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    _ok(lib, lib.sqx_silu_mul(gu.data_ptr(), m, f, act.data_ptr(), _s()))
    assert lib.sqx_int4_linear_silu_fits(m, n, f) == 1
    if m == 1:
        ks = lib.sqx_int4_linear_default_kslices(m, n, f)  # the GEMV the fused kernel runs
        _ok(lib, lib.sqx_int4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), None, 0, act.data_ptr(), 1, y1.data_ptr(), None,
                                     m, n, f, group, ks, _s()))
    else:
        nb = lib.sqx_int4_skinny_workspace_bytes(m, n, f, 0)
        ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=DEV)
        _ok(lib, lib.sqx_int4_skinny(tw.wt.data_ptr(), tw.st.data_ptr(), None, 0, act.data_ptr(), 1, y1.data_ptr(), None,
                                     m, n, f, group, -1, 0, 0, 0, ws.data_ptr() if nb > 0 else None, nb, _s()))
    _ok(lib, lib.sqx_int4_linear_silu(tw.wt.data_ptr(), tw.st.data_ptr(), gu.data_ptr(), y2.data_ptr(), m, n, f, group,
                                      0, _s()))
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    if lib.sqx_int4_prologue_fits(m, f):  # explicit waves: the GEMV with the workgroup's copy
        ks = 4
        _ok(lib, lib.sqx_int4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), None, 0, act.data_ptr(), 1, y1.data_ptr(), None,
                                     m, n, f, group, ks, _s()))
        _ok(lib, lib.sqx_int4_linear_silu(tw.wt.data_ptr(), tw.st.data_ptr(), gu.data_ptr(), y2.data_ptr(), m, n, f,
                                          group, ks, _s()))
        torch.cuda.synchronize()
        assert torch.equal(y1, y2)


def _rows_linear(lib, tw, x, m, n, k, group):
    """The linear the fused forms run: the one-row GEMV (m = 1) or the multi-row GEMV (variant 2)."""
    y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    if m == 1:
        ks = lib.sqx_int4_linear_default_kslices(1, n, k)
        _ok(lib, lib.sqx_int4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), None, 0, x.data_ptr(), 1, y.data_ptr(), None,
                                     1, n, k, group, ks, _s()))
    else:
        _ok(lib, lib.sqx_int4_skinny(tw.wt.data_ptr(), tw.st.data_ptr(), None, 0, x.data_ptr(), 1, y.data_ptr(), None,
                                     m, n, k, group, 2, 0, 0, 1, None, 0, _s()))
    return y


@pytest.mark.parametrize("n,k,group,silu,m", [(4096, 4096, 128, False, 1), (4096, 14336, 128, True, 1),
                                              (1000, 1056, 32, False, 1), (200, 2048, 64, True, 1),
                                              (4096, 4096, 128, False, 2), (4096, 14336, 128, True, 3),
                                              (4096, 14336, 128, True, 4), (1000, 1056, 32, False, 4),
                                              (200, 2048, 64, True, 8), (4096, 4096, 128, False, 7)])
def test_linear_residual_equals_two_calls(lib, n, k, group, silu, m):
    """sqx_int4_linear_residual / _silu_residual: the residual stream bit for bit as the linear they run
    (the one-row GEMV, or for 2..8 rows the multi-row GEMV) followed by the bf16 add, and the sums of
    squares per row and 16 outputs against float64 (fp32 sums of 16 squares: 16 roundings of at most
    2**-24 of the sum)."""
    print_case("linear+residual", n, k, group, silu, m)
    tw = _tiled(n, k, group, seed=n + k)
    g = torch.Generator().manual_seed(n + m)
    x = (torch.randn(m, 2 * k if silu else k, generator=g) * 2).bfloat16().to(DEV)
    res = (torch.randn(m, n, generator=g) * 3).bfloat16().to(DEV)
    act = torch.empty(m, k, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    nt = -(-n // 16)
    ss = torch.full((m, nt), float("nan"), dtype=torch.float32, device=DEV)
    src = x
    if silu:
        _ok(lib, lib.sqx_silu_mul(x.data_ptr(), m, k, act.data_ptr(), _s()))
        src = act
    y = _rows_linear(lib, tw, src, m, n, k, group)
    fn = lib.sqx_int4_linear_silu_residual if silu else lib.sqx_int4_linear_residual
    gain = (1 + 0.1 * torch.randn(n, generator=g)).bfloat16().to(DEV)
    hg = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    _ok(lib, fn(tw.wt.data_ptr(), tw.st.data_ptr(), x.data_ptr(), res.data_ptr(), out.data_ptr(), ss.data_ptr(),
                gain.data_ptr(), hg.data_ptr(), m, n, k, group, 0, _s()))
    torch.cuda.synchronize()
    want = (res.float() + y.float()).bfloat16()  # the reference's bf16 add
    assert torch.equal(out, want)
    assert torch.equal(hg, (want.float() * gain.float()).bfloat16())  # bf16(h * gain): one rounding
    h = torch.zeros(m, nt * 16, dtype=torch.float64)
    h[:, :n] = out.cpu().double()
    ref = (h * h).view(m, nt, 16).sum(2)
    got = ss.cpu().double()
    assert torch.isfinite(got).all()
    assert float(((got - ref).abs() / (16 * 2.0**-24 * ref + 1e-30)).max()) <= 1.0


@pytest.mark.parametrize("n,k,group", [(6144, 4096, 128), (28672, 4096, 128), (1000, 1056, 32), (40000, 4096, 128)])
def test_linear_rmsnorm_sumsq(lib, n, k, group):
    """sqx_int4_linear_rmsnorm_sumsq against sqx_rmsnorm then sqx_int4_linear (the same norm with the
    sum of squares in another order), with the sums as sqx_int4_linear_residual leaves them: the
    normalised row within one bf16 ulp, so y within the linear bar of the two-call result."""
    from tests.test_gpu_int4 import _check_linear

    from oracle import quant_ref as R
    from scratch_llm_amd.quant import int4_group as i4

    print_case("linear+rmsnorm from sums", n, k, group)
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(n + group)) * 0.05).to(DEV)
    q, sc = i4.quantize_groupwise_int4(w, group)
    tw = i4.tile_int4(q, sc, None, group)
    del w
    g = torch.Generator().manual_seed(k + n)
    h = (torch.randn(1, k, generator=g) * 2).bfloat16().to(DEV)
    gain = (1 + 0.1 * torch.randn(k, generator=g)).bfloat16().to(DEV)
    nt = -(-k // 16)
    hp = torch.zeros(nt * 16, dtype=torch.float32)
    hp[:k] = h.cpu().float()[0]
    ss = (hp * hp).view(nt, 16).sum(1).to(DEV)  # fp32 tile sums, as the residual epilogue writes them
    hn = torch.empty(1, k, dtype=torch.bfloat16, device=DEV)
    y1, y2 = (torch.empty(1, n, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    _ok(lib, lib.sqx_rmsnorm(h.data_ptr(), None, gain.data_ptr(), 1e-5, 1, k, None, hn.data_ptr(), _s()))
    _ok(lib, lib.sqx_int4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), None, 0, hn.data_ptr(), 1, y1.data_ptr(), None, 1, n,
                                 k, group, 0, _s()))
    _ok(lib, lib.sqx_int4_linear_rmsnorm_sumsq(tw.wt.data_ptr(), tw.st.data_ptr(), h.data_ptr(), ss.data_ptr(), nt,
                                               gain.data_ptr(), 1e-5, y2.data_ptr(), 1, n, k, group, 0, _s()))
    torch.cuda.synchronize()
    if n <= 28672:  # float64 product of the two-call form's normalised row and the dequantized weight
        w_eff = R.round_bf16(R.dequantize_groupwise_int4(q.cpu().numpy(), sc.cpu().numpy(), group))
        y_ref = R.linear_f64(hn.float().cpu().numpy(), w_eff)
        _check_linear(y2, y_ref, f"rmsnorm from sums {k}->{n}")
        _check_linear(y1, y_ref, f"plain one-row linear {k}->{n}")  # at 28672 rows the 8-wave form
    d = (y1.float() - y2.float()).abs()
    assert float(d.max()) <= 2.0**-6 * float(y1.float().abs().max())


@pytest.mark.parametrize("n,k,group,m", [(6144, 4096, 128, 1), (28672, 4096, 128, 1), (128256, 4096, 128, 1),
                                         (1000, 1056, 32, 1), (6144, 4096, 128, 2), (28672, 4096, 128, 4),
                                         (128256, 4096, 128, 3), (1000, 1024, 32, 8)])
def test_linear_rowscale_sumsq(lib, n, k, group, m):
    """sqx_int4_linear_rowscale_sumsq: RMSNorm's row factor applied to the product of bf16(h * gain)
    against the oracle: the float64 product of the reference's normalised row bf16(h * r * gain) and the
    bf16-cast dequantized weight, at the gate/up (8-wave form), qkv and lm_head shapes. Max-abs-rel
    1e-2, and elementwise the bound the roundings give: the two sides round each activation at
    different points (each within 2**-9, so 2**-8 apart), the reference rounds each weight to bf16
    (2**-9), each output is rounded to bf16 (2**-9 each side): |y - y_ref| <= 2**-7 sum_k |w_k a_k| +
    2**-8 |y_ref|."""
    from oracle import quant_ref as R
    from scratch_llm_amd.quant import int4_group as i4

    print_case("linear rowscale sums", n, k, group, m)
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(n + group)) * 0.05).to(DEV)
    q, sc = i4.quantize_groupwise_int4(w, group)
    tw = i4.tile_int4(q, sc, None, group)
    del w
    g = torch.Generator().manual_seed(k + n + m)
    h = (torch.randn(m, k, generator=g) * 2 * torch.linspace(0.5, 4, m)[:, None]).bfloat16()  # rows of other scales
    gain = (1 + 0.1 * torch.randn(k, generator=g)).bfloat16()
    nt = -(-k // 16)
    hp = torch.zeros(m, nt * 16, dtype=torch.float32)
    hp[:, :k] = h.float()
    ss = (hp * hp).view(m, nt, 16).sum(2).contiguous().to(DEV)
    hg = (h.float() * gain.float()).bfloat16().to(DEV)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    _ok(lib, lib.sqx_int4_linear_rowscale_sumsq(tw.wt.data_ptr(), tw.st.data_ptr(), hg.data_ptr(), ss.data_ptr(), nt,
                                                1e-5, y.data_ptr(), m, n, k, group, 0, _s()))
    torch.cuda.synchronize()
    hn = D.rmsnorm(h, gain, 1e-5)  # the reference's normalised rows (bf16)
    rows = torch.arange(0, n, max(1, n // 8192))
    w_eff = R.round_bf16(R.dequantize_groupwise_int4(q[rows.to(DEV)].cpu().numpy(), sc[rows.to(DEV)].cpu().numpy(), group))
    a = hn.float().numpy().astype(np.float64)
    y_ref = R.linear_f64(a, w_eff)
    got = y[:, rows.to(DEV)].float().cpu().numpy().astype(np.float64)
    err = np.abs(got - y_ref)
    assert float(err.max() / np.abs(y_ref).max()) <= 1e-2
    bound = 2.0**-7 * (np.abs(a) @ np.abs(w_eff.astype(np.float64)).T) + 2.0**-8 * np.abs(y_ref) + 1e-30
    assert float((err / bound).max()) <= 1.0, f"rowscale {k}->{n}: {float((err / bound).max()):.2f}x the bound"


@pytest.mark.parametrize("dff,k,m", [(14336, 4096, 1), (2048, 1024, 1), (1024, 4096, 1), (14336, 4096, 2),
                                      (2048, 1024, 3), (1024, 4096, 4), (1024, 1024, 6), (512, 1024, 8)])
def test_rowscale_swiglu_equals_two_calls(lib, dff, k, m):
    """sqx_int4_linear_rowscale_swiglu == sqx_int4_linear_rowscale_sumsq on the same weight (gate and up
    rows alternating in groups of 8) followed by sqx_silu_mul_pairs8, bit for bit, and that SiLU of the
    pairs == sqx_silu_mul of the [g | u] row, bit for bit: the Llama gate/up at one row (1792 tiles,
    the 8-waves-per-SIMD form), smaller one-row grids (under 1024 tiles) and 2..8 rows (the multi-row
    GEMV, one and two row groups)."""
    from scratch_llm_amd.quant import int4_group as i4

    print_case("rowscale swiglu", dff, k, m)
    gen = torch.Generator().manual_seed(dff + k + m)
    w1 = torch.randn(dff, k, generator=gen) * 0.05
    w3 = torch.randn(dff, k, generator=gen) * 0.05
    w = torch.stack([w1.view(-1, 8, k), w3.view(-1, 8, k)], 1).reshape(2 * dff, k).to(DEV)
    q, sc = i4.quantize_groupwise_int4(w, 128)
    tw = i4.tile_int4(q, sc, None, 128)
    del w
    h = (torch.randn(m, k, generator=gen) * 2).bfloat16()
    gain = (1 + 0.1 * torch.randn(k, generator=gen)).bfloat16()
    nt = k // 16
    ss = (h.float() * h.float()).view(m, nt, 16).sum(2).contiguous().to(DEV)
    hg = (h.float() * gain.float()).bfloat16().to(DEV)
    n = 2 * dff
    gu = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    want = torch.empty(m, dff, dtype=torch.bfloat16, device=DEV)
    got = torch.empty(m, dff, dtype=torch.bfloat16, device=DEV)
    _ok(lib, lib.sqx_int4_linear_rowscale_sumsq(tw.wt.data_ptr(), tw.st.data_ptr(), hg.data_ptr(), ss.data_ptr(), nt,
                                                1e-5, gu.data_ptr(), m, n, k, 128, 0, _s()))
    _ok(lib, lib.sqx_silu_mul_pairs8(gu.data_ptr(), m, dff, want.data_ptr(), _s()))
    _ok(lib, lib.sqx_int4_linear_rowscale_swiglu(tw.wt.data_ptr(), tw.st.data_ptr(), hg.data_ptr(), ss.data_ptr(), nt,
                                                 1e-5, got.data_ptr(), m, n, k, 128, 0, _s()))
    # the pairs' SiLU against the [g | u] kernel on the de-interleaved row
    flat = gu.view(m, dff // 8, 2, 8)
    side = torch.cat([flat[:, :, 0].reshape(m, dff), flat[:, :, 1].reshape(m, dff)], 1).contiguous()
    ref = torch.empty(m, dff, dtype=torch.bfloat16, device=DEV)
    _ok(lib, lib.sqx_silu_mul(side.data_ptr(), m, dff, ref.data_ptr(), _s()))
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(want, ref), "silu of the 8-row pairs != silu of the [g | u] row"
    assert torch.equal(got, want), f"{k}->{n} m={m}: epilogue != two calls"


@pytest.mark.parametrize("dff,k,m", [(14336, 4096, 1), (14336, 4096, 2), (14336, 4096, 8), (14336, 4096, 16),
                                      (14336, 4096, 33), (14336, 4096, 64), (1024, 1024, 3), (1024, 1024, 20)])
def test_linear_swiglu_equals_two_calls(lib, dff, k, m):
    """sqx_int4_linear_swiglu == the library's linear for the shape (sqx_int4_linear at one row,
    sqx_int4_skinny without a workspace above) followed by sqx_silu_mul_pairs8, bit for bit: the
    one-row GEMV, the multi-row GEMV and both row-tiled kernels at the Llama gate/up shape."""
    from scratch_llm_amd import _lib
    from scratch_llm_amd.quant import int4_group as i4

    print_case("linear swiglu", dff, k, m)
    gen = torch.Generator(device=DEV).manual_seed(dff + k + m)
    q, sc = i4.quantize_groupwise_int4(torch.randn(2 * dff, k, generator=gen, device=DEV) * 0.05, 128)
    tw = i4.tile_int4(q, sc, None, 128)
    x = torch.randn(m, k, generator=gen, device=DEV).to(torch.bfloat16)
    n = 2 * dff
    gu = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    want = torch.empty(m, dff, dtype=torch.bfloat16, device=DEV)
    got = torch.empty(m, dff, dtype=torch.bfloat16, device=DEV)
    if m == 1:
        _ok(lib, lib.sqx_int4_linear(tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32, x.data_ptr(),
                                     _lib.DTYPE_BF16, gu.data_ptr(), None, 1, n, k, 128, 0, _s()))
    else:
        _ok(lib, lib.sqx_int4_skinny(tw.wt.data_ptr(), tw.st.data_ptr(), None, _lib.DTYPE_F32, x.data_ptr(),
                                     _lib.DTYPE_BF16, gu.data_ptr(), None, m, n, k, 128, -1, 0, 0, 0, None, 0, _s()))
    _ok(lib, lib.sqx_silu_mul_pairs8(gu.data_ptr(), m, dff, want.data_ptr(), _s()))
    _ok(lib, lib.sqx_int4_linear_swiglu(tw.wt.data_ptr(), tw.st.data_ptr(), x.data_ptr(), got.data_ptr(), m, n, k,
                                        128, _s()))
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, want), f"{k}->{n} m={m}: epilogue != two calls"


def test_rowscale_swiglu_refuses(lib):
    """Rows that are not whole 16-row tiles, or more rows than the fused forms take, are refused."""
    rc = lib.sqx_int4_linear_rowscale_swiglu(None, None, None, None, 64, 1e-5, None, 1, 1000, 1024, 128, 0, None)
    assert rc != 0
    rc = lib.sqx_int4_linear_rowscale_swiglu(None, None, None, None, 64, 1e-5, None, 9, 2048, 1024, 128, 0, None)
    assert rc != 0 and "1..8 rows" in lib.sqx_last_error().decode()


@pytest.mark.parametrize("H,Hkv,T,length,sums,m", [(32, 8, 2048, 2047, True, 1), (32, 8, 2048, 0, False, 1),
                                                    (8, 2, 100, 140, True, 1), (16, 16, 64, 37, False, 1),
                                                    (32, 8, 2048, 2040, True, 4), (8, 2, 100, 50, False, 2),
                                                    (16, 16, 64, 37, True, 8)])
def test_linear_rope_kv_equals_two_calls(lib, H, Hkv, T, length, sums, m):
    """sqx_int4_linear_rope_kv == the linear (sqx_int4_linear_rowscale_sumsq, or the plain one-row /
    multi-row GEMV) followed by sqx_rope_kv on its output, bit for bit: the rotated q, and the cache
    rows (only row min(length, T - 1) of each slot changes; rows of m slots sit at positions length,
    length + 3, ...), at a full slot and at position 0 too."""
    from scratch_llm_amd.quant import int4_group as i4

    print_case("linear rope kv", H, Hkv, T, length, sums, m)
    hd, k = 128, 4096 if H == 32 else 1024
    n = (H + 2 * Hkv) * hd
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(n + k)) * 0.05).to(DEV)
    q, sc = i4.quantize_groupwise_int4(w)
    tw = i4.tile_int4(q, sc)
    del w
    g = torch.Generator().manual_seed(H + T + m)
    x = (torch.randn(m, k, generator=g) * 2).bfloat16().to(DEV)
    nt = k // 16
    ss = (torch.rand(m, nt, generator=g) * 50).to(DEV) if sums else None
    lens = [length + 3 * r for r in range(m)]
    ctx = max(T, max(lens) + 1) + 8
    cos, sin = (t.to(DEV) for t in D.rope_tables(hd, ctx, 10000.0))
    ln = torch.tensor(lens, dtype=torch.int32, device=DEV)
    cache = torch.randn(2, m, Hkv, T, hd, generator=g).bfloat16().to(DEV)
    # the two-call form
    if sums:
        y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        _ok(lib, lib.sqx_int4_linear_rowscale_sumsq(tw.wt.data_ptr(), tw.st.data_ptr(), x.data_ptr(), ss.data_ptr(), nt,
                                                    1e-5, y.data_ptr(), m, n, k, 128, 0, _s()))
    else:
        y = _rows_linear(lib, tw, x, m, n, k, 128)
    q2 = torch.empty(m, H, hd, dtype=torch.bfloat16, device=DEV)
    kc2, vc2 = cache[0].clone(), cache[1].clone()
    _ok(lib, lib.sqx_rope_kv(y.data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx, m, H, Hkv, hd, T,
                             q2.data_ptr(), kc2.data_ptr(), vc2.data_ptr(), _s()))
    # the fused form
    q1 = torch.empty(m, H * hd, dtype=torch.bfloat16, device=DEV)
    kc1, vc1 = cache[0].clone(), cache[1].clone()
    _ok(lib, lib.sqx_int4_linear_rope_kv(tw.wt.data_ptr(), tw.st.data_ptr(), x.data_ptr(),
                                         None if ss is None else ss.data_ptr(), nt, 1e-5, ln.data_ptr(), cos.data_ptr(),
                                         sin.data_ptr(), ctx, H, Hkv, T, q1.data_ptr(), kc1.data_ptr(), vc1.data_ptr(),
                                         m, n, k, 128, 0, _s()))
    torch.cuda.synchronize()
    assert torch.equal(q1.view(m, H, hd), q2)
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    for r in range(m):
        slot = min(lens[r], T - 1)
        assert not torch.equal(kc1[r, :, slot], cache[0][r, :, slot])


def _partials(lib, q, lengths, k, v, B, H, Hkv, T, cos=None, sin=None, rope_rows=0, ks=None, vs=None):
    """sqx_decode_attention_partials into a fresh workspace (NaN-filled: only what it writes is read)."""
    nb = lib.sqx_attn_partials_workspace_bytes(B, H, T)
    ws = torch.full((nb // 4,), float("nan"), dtype=torch.float32, device=DEV)
    _ok(lib, lib.sqx_decode_attention_partials(
        q.data_ptr(), lengths.data_ptr(), None if cos is None else cos.data_ptr(), None if sin is None else sin.data_ptr(),
        rope_rows, k.data_ptr(), v.data_ptr(), None if ks is None else ks.data_ptr(), None if vs is None else vs.data_ptr(),
        B, H, Hkv, 128, T, ws.data_ptr(), nb, _s()))
    return ws


@pytest.mark.parametrize("B,H,Hkv,T,kv8", [(1, 32, 8, 2048, False), (3, 16, 2, 300, False), (4, 8, 8, 77, False),
                                           (1, 32, 8, 2048, True), (3, 16, 8, 300, True)])
def test_attention_partials_against_float64(lib, B, H, Hkv, T, kv8):
    """The 8-wave partials (at most 8 chunks per head) merged by sqx_attn_partials_combine: softmax
    attention within 2**-8 |ref| + 1e-5 max|v| of float64, for ragged lengths (0, mid-chunk, T - 1, past
    T), bf16 and E4M3 caches."""
    from oracle import fp8_ref as F8

    print_case("attention partials", B, H, Hkv, T, kv8)
    hd = 128
    chunk = lib.sqx_attn_partials_chunk(T)
    assert chunk % 128 == 0 and -(-T // chunk) <= 8
    g = torch.Generator().manual_seed(B * 100 + T + kv8)
    lengths = ([T - 1, 0, T // 2 + 3, T + 4] * B)[:B]
    q = (torch.randn(B, H, hd, generator=g) * 2).bfloat16()
    if kv8:
        kc, vc = _valid_codes((B, Hkv, T, hd), g), _valid_codes((B, Hkv, T, hd), g)
        ks = torch.rand(Hkv, generator=g) * 0.01 + 0.001
        vs = torch.rand(Hkv, generator=g) * 0.01 + 0.001
        kdeq = torch.from_numpy(F8.e4m3_decode(kc.numpy())).double() * ks.double().view(1, Hkv, 1, 1)
        vdeq = torch.from_numpy(F8.e4m3_decode(vc.numpy())).double() * vs.double().view(1, Hkv, 1, 1)
        ksd, vsd = ks.to(DEV), vs.to(DEV)
    else:
        kc = (torch.randn(B, Hkv, T, hd, generator=g) * 2).bfloat16()
        vc = torch.randn(B, Hkv, T, hd, generator=g).bfloat16()
        kdeq, vdeq = kc.double(), vc.double()
        ksd = vsd = None
    ln = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    ws = _partials(lib, q.to(DEV), ln, kc.to(DEV), vc.to(DEV), B, H, Hkv, T, ks=ksd, vs=vsd)
    out = torch.empty(B, H * hd, dtype=torch.bfloat16, device=DEV)
    _ok(lib, lib.sqx_attn_partials_combine(ws.data_ptr(), ln.data_ptr(), B, H, T, out.data_ptr(), _s()))
    torch.cuda.synchronize()
    G = H // Hkv
    got = out.cpu().view(B, H, hd).double()
    assert torch.isfinite(got).all()
    for b in range(B):
        L = min(max(lengths[b], 0) + 1, T)
        kk = kdeq[b, :, :L].repeat_interleave(G, dim=0)
        vv = vdeq[b, :, :L].repeat_interleave(G, dim=0)
        p = torch.softmax(torch.einsum("hd,htd->ht", q[b].double(), kk) / math.sqrt(hd), dim=-1)
        want = torch.einsum("ht,htd->hd", p, vv)
        bound = 2.0**-8 * want.abs() + 1e-5 * vv.abs().max()
        assert float(((got[b] - want).abs() / bound).max()) <= 1.0, f"row {b} (L={L})"


@pytest.mark.parametrize("B,H,Hkv,T,kv8", [(1, 32, 8, 2048, False), (5, 16, 2, 300, False), (1, 32, 8, 2048, True)])
def test_attention_partials_rope_equals_two_calls(lib, B, H, Hkv, T, kv8):
    """The RoPE form of sqx_decode_attention_partials == sqx_rope_kv (the new row quantized with the
    head's scales for an E4M3 cache) then the plain form, bit for bit (partials and caches)."""
    print_case("attention partials rope", B, H, Hkv, T, kv8)
    hd, ctx = 128, T + 16
    g = torch.Generator().manual_seed(B * 7 + T + kv8)
    lengths = torch.randint(0, T, (B,), generator=g)
    lengths[0] = T - 1
    if B > 1:
        lengths[1] = 0
    if B > 2:
        lengths[2] = T + 9
    qkv = (torch.randn(B, (H + 2 * Hkv) * hd, generator=g) * 2).bfloat16().to(DEV)
    cos, sin = (t.to(DEV) for t in D.rope_tables(hd, ctx, 10000.0))
    ln = lengths.to(torch.int32).to(DEV)
    if kv8:
        cache = [_valid_codes((B, Hkv, T, hd), g).to(DEV) for _ in range(2)]
        ks = (torch.rand(Hkv, generator=g) * 0.01 + 0.004).to(DEV)
        vs = (torch.rand(Hkv, generator=g) * 0.01 + 0.004).to(DEV)
    else:
        cache = [torch.randn(B, Hkv, T, hd, generator=g).bfloat16().to(DEV) for _ in range(2)]
        ks = vs = None
    # fused: RoPE, the cache write and the partials in one launch
    kf, vf = cache[0].clone(), cache[1].clone()
    wf = _partials(lib, qkv, ln, kf, vf, B, H, Hkv, T, cos, sin, ctx, ks, vs)
    # two calls: rotate and write the row (bf16), or rotate into a bf16 scratch cache and quantize the
    # new row with the head's scales (E4M3), then the plain partials on the rotated q
    q = torch.empty(B, H * hd, dtype=torch.bfloat16, device=DEV)
    k2, v2 = cache[0].clone(), cache[1].clone()
    if kv8:
        kb = torch.zeros(B, Hkv, T, hd, dtype=torch.bfloat16, device=DEV)
        vb = torch.zeros_like(kb)
        _ok(lib, lib.sqx_rope_kv(qkv.data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx, B, H, Hkv, hd, T,
                                 q.data_ptr(), kb.data_ptr(), vb.data_ptr(), _s()))
        torch.cuda.synchronize()
        from oracle import fp8_ref as F8

        for b in range(B):
            slot = min(int(lengths[b]), T - 1)
            for t_, src, sc in ((k2, kb, ks), (v2, vb, vs)):
                row = src[b, :, slot].float().cpu().numpy()  # [Hkv, hd]
                t_[b, :, slot] = torch.from_numpy(
                    F8.e4m3_encode_sat(row / sc.cpu().numpy()[:, None].astype(np.float32))).to(DEV)
    else:
        _ok(lib, lib.sqx_rope_kv(qkv.data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx, B, H, Hkv, hd, T,
                                 q.data_ptr(), k2.data_ptr(), v2.data_ptr(), _s()))
    w2 = _partials(lib, q, ln, k2, v2, B, H, Hkv, T, ks=ks, vs=vs)
    torch.cuda.synchronize()
    assert torch.equal(kf, k2) and torch.equal(vf, v2)
    o1, o2 = (torch.empty(B, H * hd, dtype=torch.bfloat16, device=DEV) for _ in range(2))
    _ok(lib, lib.sqx_attn_partials_combine(wf.data_ptr(), ln.data_ptr(), B, H, T, o1.data_ptr(), _s()))
    _ok(lib, lib.sqx_attn_partials_combine(w2.data_ptr(), ln.data_ptr(), B, H, T, o2.data_ptr(), _s()))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


@pytest.mark.parametrize("H,Hkv,T,length,n", [(32, 8, 2048, 2047, 4096), (32, 8, 2048, 0, 4096),
                                              (32, 8, 2048, 5000, 4096), (32, 8, 300, 150, 4096),
                                              (8, 2, 1000, 700, 1024), (16, 16, 64, 63, 2048)])
def test_linear_attn_residual_equals_two_calls(lib, H, Hkv, T, length, n):
    """sqx_int4_linear_attn_residual (the combine in the o projection's activation load) ==
    sqx_attn_partials_combine then sqx_int4_linear_residual with the same k_slices, bit for bit:
    residual stream, sums of squares and bf16(h * gain); chunk counts 1, 3 and 8."""
    print_case("linear attn residual", H, Hkv, T, length, n)
    hd = 128
    k = H * hd
    tw = _tiled(n, k, 128, seed=H + T)
    g = torch.Generator().manual_seed(T + length)
    q = (torch.randn(1, H, hd, generator=g) * 2).bfloat16().to(DEV)
    kc = (torch.randn(1, Hkv, T, hd, generator=g) * 2).bfloat16().to(DEV)
    vc = torch.randn(1, Hkv, T, hd, generator=g).bfloat16().to(DEV)
    ln = torch.tensor([length], dtype=torch.int32, device=DEV)
    ws = _partials(lib, q, ln, kc, vc, 1, H, Hkv, T)
    res = (torch.randn(1, n, generator=g) * 3).bfloat16().to(DEV)
    gain = (1 + 0.1 * torch.randn(n, generator=g)).bfloat16().to(DEV)
    att = torch.empty(1, k, dtype=torch.bfloat16, device=DEV)
    nt = -(-n // 16)
    out1, out2, hg1, hg2 = (torch.empty(1, n, dtype=torch.bfloat16, device=DEV) for _ in range(4))
    ss1, ss2 = (torch.full((nt,), float("nan"), dtype=torch.float32, device=DEV) for _ in range(2))
    ksl = k // 256
    _ok(lib, lib.sqx_attn_partials_combine(ws.data_ptr(), ln.data_ptr(), 1, H, T, att.data_ptr(), _s()))
    _ok(lib, lib.sqx_int4_linear_residual(tw.wt.data_ptr(), tw.st.data_ptr(), att.data_ptr(), res.data_ptr(),
                                          out1.data_ptr(), ss1.data_ptr(), gain.data_ptr(), hg1.data_ptr(), 1, n, k, 128,
                                          ksl, _s()))
    _ok(lib, lib.sqx_int4_linear_attn_residual(tw.wt.data_ptr(), tw.st.data_ptr(), ws.data_ptr(), ln.data_ptr(), T,
                                               res.data_ptr(), out2.data_ptr(), ss2.data_ptr(), gain.data_ptr(),
                                               hg2.data_ptr(), 1, n, k, 128, ksl, _s()))
    torch.cuda.synchronize()
    assert torch.isfinite(att.float()).all()
    assert torch.equal(out1, out2)
    assert torch.equal(hg1, hg2)
    assert torch.equal(ss1, ss2)


def test_linear_attn_residual_refuses(lib):
    """The merge prologue's limits come back as SQX_E_ARG: more than two k-blocks per wave, a width
    that is not whole heads, more than one row."""
    tw = _tiled(1024, 4096, 128, seed=1)
    p = tw.wt.data_ptr()
    buf = torch.zeros(8192, dtype=torch.float32, device=DEV)
    b = buf.data_ptr()
    assert lib.sqx_int4_linear_attn_residual(p, tw.st.data_ptr(), b, b, 2048, b, b, b, None, None, 1, 1024, 4096, 128,
                                             8, _s()) == -1
    assert "two k-blocks" in lib.sqx_last_error().decode()
    assert lib.sqx_int4_linear_attn_residual(p, tw.st.data_ptr(), b, b, 2048, b, b, b, None, None, 2, 1024, 4096, 128,
                                             16, _s()) == -1


def test_residual_forms_refuse(lib):
    tw = _tiled(64, 4096, 128, seed=3)
    x = torch.zeros(9, 4096, dtype=torch.bfloat16, device=DEV)
    ss = torch.zeros(9 * 256, dtype=torch.float32, device=DEV)
    assert lib.sqx_int4_linear_residual(tw.wt.data_ptr(), tw.st.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(),
                                        ss.data_ptr(), None, None, 9, 64, 4096, 128, 0, _s()) == -1
    assert "2..8 rows" in lib.sqx_last_error().decode()
    # 160 k-blocks: k-slices of 10 blocks over 16 waves, more than the multi-row form takes
    tw20 = _tiled(64, 20480, 128, seed=4)
    x20 = torch.zeros(5, 20480, dtype=torch.bfloat16, device=DEV)
    assert lib.sqx_int4_rows_fits(5, 64, 20480, 0) == 0 and lib.sqx_int4_rows_fits(5, 64, 14336, 0) == 1
    assert lib.sqx_int4_linear_residual(tw20.wt.data_ptr(), tw20.st.data_ptr(), x20.data_ptr(), x.data_ptr(),
                                        x.data_ptr(), ss.data_ptr(), None, None, 5, 64, 20480, 128, 0, _s()) == -1
    assert "multi-row form" in lib.sqx_last_error().decode()
    assert lib.sqx_int4_linear_residual(tw.wt.data_ptr(), tw.st.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(),
                                        ss.data_ptr(), x.data_ptr(), None, 1, 64, 4096, 128, 0, _s()) == -1
    assert "go together" in lib.sqx_last_error().decode()
    assert lib.sqx_int4_linear_rowscale_sumsq(tw.wt.data_ptr(), tw.st.data_ptr(), x.data_ptr(), ss.data_ptr(), 255,
                                              1e-5, x.data_ptr(), 1, 64, 4096, 128, 0, _s()) == -1
    assert "sums of squares" in lib.sqx_last_error().decode()
    assert lib.sqx_int4_linear_rmsnorm_sumsq(tw.wt.data_ptr(), tw.st.data_ptr(), x.data_ptr(), ss.data_ptr(), 255,
                                             x.data_ptr(), 1e-5, x.data_ptr(), 1, 64, 4096, 128, 0, _s()) == -1
    assert "sums of squares" in lib.sqx_last_error().decode()


def test_fused_prologue_refuses_what_does_not_fit(lib):
    assert lib.sqx_int4_prologue_fits(8, 4096) == 0  # 8 rows of 4096 exceed the 64 KiB copy
    assert lib.sqx_int4_prologue_fits(3, 14336) == 0
    assert lib.sqx_int4_prologue_fits(9, 128) == 0
    tw = _tiled(64, 4096, 128, seed=1)
    x = torch.zeros(8, 4096, dtype=torch.bfloat16, device=DEV)
    assert lib.sqx_int4_linear_rmsnorm(tw.wt.data_ptr(), tw.st.data_ptr(), x.data_ptr(), None, x.data_ptr(), 1e-5, None,
                                       x.data_ptr(), 8, 64, 4096, 128, 0, _s()) == -1


def test_attention_rejects_bad_shapes(lib):
    ws = torch.empty(16, dtype=torch.float32, device=DEV)
    assert lib.sqx_decode_attention(ws.data_ptr(), ws.data_ptr(), ws.data_ptr(), ws.data_ptr(), 1, 32, 8, 64, 16, ws.data_ptr(),
                                    ws.data_ptr(), 64, _s()) == -1
    assert lib.sqx_decode_attention(ws.data_ptr(), ws.data_ptr(), ws.data_ptr(), ws.data_ptr(), 1, 48, 8, 128, 16,
                                    ws.data_ptr(), ws.data_ptr(), 64, _s()) == -1
    assert lib.sqx_decode_attention(ws.data_ptr(), ws.data_ptr(), ws.data_ptr(), ws.data_ptr(), 4, 32, 8, 128, 2048,
                                    ws.data_ptr(), ws.data_ptr(), 64, _s()) == -3


@pytest.mark.parametrize("B,F", [(1, 14336), (5, 96), (64, 2048), (3, 100)])  # F = 100: the two-element kernel
def test_silu_mul(lib, B, F):
    print_case("silu_mul", B, F)
    g = torch.Generator().manual_seed(F)
    gu = (torch.randn(B, 2 * F, generator=g) * 4).bfloat16()
    gu[0, :4] = torch.tensor([0.0, -0.0, 80.0, -80.0]).bfloat16()
    out = torch.empty(B, F, dtype=torch.bfloat16, device=DEV)
    _ok(lib, lib.sqx_silu_mul(gu.to(DEV).data_ptr(), B, F, out.data_ptr(), _s()))
    torch.cuda.synchronize()
    gg, uu = gu[:, :F].double(), gu[:, F:].double()
    want = gg * torch.sigmoid(gg) * uu
    err = (out.cpu().double() - want).abs()
    assert bool((err <= 2.0**-8 * want.abs() + 1e-30).all())


def test_embed_argmax_advance(lib):
    print_case("embed/argmax/advance")
    V, d, B = 1000, 256, 5
    table = torch.randn(V, d).bfloat16()
    tok = torch.tensor([0, 999, 17, -1, 1000], dtype=torch.int32)
    td = table.to(DEV)
    out = torch.empty(B, d, dtype=torch.bfloat16, device=DEV)
    _ok(lib, lib.sqx_embed(td.data_ptr(), V, tok.to(DEV).data_ptr(), B, d, out.data_ptr(), _s()))
    torch.cuda.synchronize()
    o = out.cpu()
    assert torch.equal(o[:3], table[tok[:3].long()])
    assert not o[3:].any()  # out-of-range ids give zero rows
    # argmax: first index of the maximum, NaN wins, at the config-5 vocabulary
    for Vv in (128256, 7, 300):
        lg = torch.randn(6, Vv).bfloat16()
        lg[1, :] = 0.0  # all tied -> 0
        lg[2, Vv // 3] = 100.0
        lg[2, Vv - 1] = 100.0  # tie -> the first
        lg[3, Vv // 2] = float("nan")
        lg[3, Vv - 1] = float("nan")
        lg[4, :] = float("-inf")
        nt = torch.empty(6, dtype=torch.int32, device=DEV)
        nb = lib.sqx_argmax_workspace_bytes(6, Vv)
        ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
        _ok(lib, lib.sqx_argmax(lg.to(DEV).data_ptr(), 6, Vv, nt.data_ptr(), ws.data_ptr(), nb, _s()))
        if Vv == 128256:  # a row split over many workgroups: the max in the last one, and a tie across two
            lg2 = torch.zeros(2, Vv).bfloat16()
            lg2[0, Vv - 3] = 5.0
            lg2[1, 10] = 7.0
            lg2[1, Vv - 9] = 7.0
            nt2 = torch.empty(2, dtype=torch.int32, device=DEV)
            _ok(lib, lib.sqx_argmax(lg2.to(DEV).data_ptr(), 2, Vv, nt2.data_ptr(), ws.data_ptr(), nb, _s()))
            torch.cuda.synchronize()
            assert nt2.cpu().tolist() == [Vv - 3, 10]
        torch.cuda.synchronize()
        assert nt.cpu().tolist() == lg.float().argmax(dim=-1).tolist()
    # advance: named values of tests/test_batched_cache.py:91-103
    ln = torch.tensor([4, 2, 0], dtype=torch.int32, device=DEV)
    act = torch.tensor([1, 0, 1], dtype=torch.uint8, device=DEV)
    _ok(lib, lib.sqx_advance(ln.data_ptr(), act.data_ptr(), 3, _s()))
    torch.cuda.synchronize()
    assert ln.cpu().tolist() == [5, 2, 1]
    _ok(lib, lib.sqx_advance(ln.data_ptr(), None, 3, _s()))
    torch.cuda.synchronize()
    assert ln.cpu().tolist() == [6, 3, 2]


# ---------------------------------------------------------------------------------------------
# the whole step
# ---------------------------------------------------------------------------------------------
SMALL = dict(vocab=1000, d_model=1024, n_layers=2, n_heads=8, n_kv_heads=2, d_ff=2048)


@pytest.fixture(scope="module")
def small():
    from scratch_llm_amd.decode import DecodeConfig, Int4DecodeLM

    p = D.random_params(**SMALL, seed=11, std=0.05)
    cfg = DecodeConfig(vocab_size=SMALL["vocab"], d_model=SMALL["d_model"], n_layers=SMALL["n_layers"],
                       n_heads=SMALL["n_heads"], n_kv_heads=SMALL["n_kv_heads"], d_ff=SMALL["d_ff"],
                       context_length=64)
    model = Int4DecodeLM.from_state_dict(cfg, lambda n: p[n], DEV)
    refs = {dt: D.int4_model(p, n_layers=cfg.n_layers, n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads,
                             context_length=cfg.context_length, dtype=dt) for dt in (torch.bfloat16, torch.float32)}
    return model, refs


def _run_and_compare(model, refs, B, steps, seed, max_ctx=48):
    g = torch.Generator().manual_seed(seed)
    st = model.new_state(B, max_ctx)
    caches = {dt: D.RefCache.empty(r, B, max_ctx, dt) for dt, r in refs.items()}
    tok = torch.randint(0, model.cfg.vocab_size, (B,), generator=g)
    for t in range(steps):
        print_case("decode step", f"B={B}", f"t={t}")
        nxt = model.step(st, tok)
        torch.cuda.synchronize()
        got = st.logits.float().cpu()
        l16 = D.decode_step(refs[torch.bfloat16], caches[torch.bfloat16], tok, torch.bfloat16).float()
        l32 = D.decode_step(refs[torch.float32], caches[torch.float32], tok, torch.float32)
        scale = float(l32.abs().max())
        e_hip = float((got - l32).abs().max())
        e_ref = float((l16 - l32).abs().max())
        assert e_hip <= 2 * e_ref + 2.0**-9 * scale, f"t={t}: |hip-f32| {e_hip:.4g} vs |bf16 ref-f32| {e_ref:.4g}"
        top2 = l32.topk(2, dim=-1).values
        sure = (top2[:, 0] - top2[:, 1]) > 4 * e_hip
        picks = nxt.cpu().long()
        assert torch.equal(picks[sure], l32.argmax(-1)[sure]), f"t={t}: greedy picks differ"
        assert st.lengths.cpu().tolist() == caches[torch.float32].lengths.tolist()
        tok = picks
    return st


@pytest.mark.parametrize("B", [1, 3, 64])
def test_decode_step_matches_reference(small, B):
    model, refs = small
    _run_and_compare(model, refs, B, steps=6 if B < 64 else 3, seed=B)


@pytest.mark.parametrize("B", [1, 2, 4, 5])
def test_fused_step_equals_unfused_step(small, B):
    """The norm folded into the GEMV's LDS copy (fuse_norm) is bit-identical at one row; at more rows
    the two-call form's linear may be the multi-row GEMV, which sums in another order, so the logits
    agree to the bf16 rounding of the step."""
    model, _ = small
    print_case("fused vs unfused step", B)
    try:
        model.fuse_norm_sums = False  # its norm adds the sum of squares in another order (tested below)
        for fuse_norm in (False, True):
            a, b = model.new_state(B, 32), model.new_state(B, 32)
            tok = torch.arange(B) * 97 % model.cfg.vocab_size
            for t in range(4):
                model.fuse_norm = fuse_norm
                model.step(a, tok if t == 0 else None)
                model.fuse_norm = False
                model.step(b, tok if t == 0 else None)
                torch.cuda.synchronize()
                if fuse_norm and B > 1:
                    scale = float(b.logits.float().abs().max())
                    assert float((a.logits.float() - b.logits.float()).abs().max()) <= 2.0**-5 * scale, f"step {t}"
                    b.tokens.copy_(a.tokens)  # follow the same tokens
                    continue
                assert torch.equal(a.logits, b.logits), f"fuse_norm={fuse_norm} step {t}"
                assert torch.equal(a.tokens, b.tokens)
            if not (fuse_norm and B > 1):
                assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)
    finally:
        model.fuse_norm, model.fuse_norm_sums = False, True


@pytest.mark.parametrize("B", [20, 64])
def test_split_partials_norm_step_equals_reduce_step(small, B):
    """The K-split o / down partials added by the norm and the q|k|v partials added by the attention
    kernel (no reduce launches) change no bit of the step or the cache: at B = 20 o, down and q|k|v
    split in the small model, at B = 64 down does."""
    from scratch_llm_amd import _lib

    model, _ = small
    lib = _lib.load()
    cfg = model.cfg
    splits = [lib.sqx_int4_skinny_default_splits(B, cfg.d_model, cfg.n_heads * cfg.head_dim),
              lib.sqx_int4_skinny_default_splits(B, cfg.d_model, cfg.d_ff),
              lib.sqx_int4_skinny_default_splits(B, (cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim, cfg.d_model)]
    assert max(splits) >= 2, splits
    assert B != 20 or min(splits) >= 2, splits
    print_case("split partials norm step", B, splits)
    a, b = model.new_state(B, 32), model.new_state(B, 32)
    tok = torch.arange(B) * 31 % cfg.vocab_size
    try:
        for t in range(3):
            model.fuse_split_norm = model.fuse_qkv_parts = True
            model.step(a, tok if t == 0 else None)
            model.fuse_split_norm = model.fuse_qkv_parts = False
            model.step(b, tok if t == 0 else None)
            torch.cuda.synchronize()
            assert torch.equal(a.logits, b.logits), f"step {t}"
            assert torch.equal(a.tokens, b.tokens)
        assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)
    finally:
        model.fuse_split_norm = model.fuse_qkv_parts = True


def test_rmsnorm_partials_equals_reduce_then_norm(lib):
    """sqx_int4_skinny_partials + sqx_rmsnorm_partials == sqx_int4_skinny (its own reduce) + sqx_rmsnorm,
    bit for bit, and the partials form refuses a shape whose launch does not split."""
    m, n, k = 48, 4096, 14336
    S = lib.sqx_int4_skinny_default_splits(m, n, k)
    print_case("rmsnorm partials", m, n, k, S)
    assert S >= 2
    tw = _tiled(n, k, 128, seed=9)
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(m, k, generator=g)).bfloat16().to(DEV)
    res = (torch.randn(m, n, generator=g) * 2).bfloat16().to(DEV)
    gain = (1 + 0.1 * torch.randn(n, generator=g)).bfloat16().to(DEV)
    nb = lib.sqx_int4_skinny_workspace_bytes(m, n, k, 0)
    ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    h1, h2, o1, o2 = (torch.empty(m, n, dtype=torch.bfloat16, device=DEV) for _ in range(4))
    _ok(lib, lib.sqx_int4_skinny(tw.wt.data_ptr(), tw.st.data_ptr(), None, 0, x.data_ptr(), 1, y.data_ptr(), None, m, n,
                                 k, 128, -1, 0, 0, 0, ws.data_ptr(), nb, _s()))
    _ok(lib, lib.sqx_rmsnorm(res.data_ptr(), y.data_ptr(), gain.data_ptr(), 1e-5, m, n, h1.data_ptr(), o1.data_ptr(),
                             _s()))
    _ok(lib, lib.sqx_int4_skinny_partials(tw.wt.data_ptr(), tw.st.data_ptr(), None, 0, x.data_ptr(), 1, m, n, k, 128,
                                          ws.data_ptr(), nb, _s()))
    _ok(lib, lib.sqx_rmsnorm_partials(res.data_ptr(), ws.data_ptr(), S, gain.data_ptr(), 1e-5, m, n, h2.data_ptr(),
                                      o2.data_ptr(), _s()))
    torch.cuda.synchronize()
    assert torch.equal(h1, h2) and torch.equal(o1, o2)
    assert lib.sqx_int4_skinny_default_splits(4, 6144, 4096) == 1
    assert lib.sqx_int4_skinny_partials(tw.wt.data_ptr(), tw.st.data_ptr(), None, 0, x.data_ptr(), 1, 4, 6144, 4096,
                                        128, ws.data_ptr(), nb, _s()) == -1
    assert "does not split" in lib.sqx_last_error().decode()


@pytest.mark.parametrize("B", [1, 2, 4, 8])
def test_norm_sums_step_matches_reference_both_ways(small, B):
    """The step with the norms folded into the residual epilogues (the default: the one-row GEMV at one
    row, the multi-row GEMV at 2..8 rows) and without: both within the reference bar of the step
    oracle at every step (_run_and_compare), from the same tokens."""
    model, refs = small
    from scratch_llm_amd import _lib

    lib = _lib.load()
    cfg = model.cfg
    if B > 1:  # the small model's linears all fit the multi-row form, so the default step is the fused one
        assert lib.sqx_int4_rows_fits(B, cfg.d_model, cfg.d_ff, 0) == 1
    try:
        for flag in (True, False):
            model.fuse_norm_sums = flag
            _run_and_compare(model, refs, B, steps=5, seed=11 + B)
    finally:
        model.fuse_norm_sums = True


def test_graph_replays_equal_eager_steps(small):
    """A captured step replayed token after token gives the bits of eager steps from the same state."""
    model, _ = small
    print_case("graph replay")
    B, steps = 4, 5
    a, b = model.new_state(B, 32), model.new_state(B, 32)
    tok = torch.tensor([5, 17, 300, 999])
    a.set_tokens(tok, model.cfg.vocab_size)
    b.set_tokens(tok, model.cfg.vocab_size)
    graph = model.capture(b)
    for t in range(steps):
        model.step(a)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(a.logits, b.logits), f"replay {t}"
        assert torch.equal(a.tokens, b.tokens) and torch.equal(a.lengths, b.lengths)
    assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)
    assert b.lengths.cpu().tolist() == [steps] * B


@pytest.mark.parametrize("B", [2, 5])
def test_fused_rows_graph_replays_equal_eager_steps(small, B):
    """The 2..8-row step without norm launches (residual epilogues, row factors, RoPE in the qkv
    epilogue on the multi-row GEMV) captured and replayed equals eager steps bit for bit."""
    model, _ = small
    print_case("graph replay fused rows", B)
    a, b = model.new_state(B, 32), model.new_state(B, 32)
    tok = torch.arange(B) * 131 % model.cfg.vocab_size
    a.set_tokens(tok, model.cfg.vocab_size)
    b.set_tokens(tok, model.cfg.vocab_size)
    graph = model.capture(b)
    for t in range(5):
        model.step(a)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(a.logits, b.logits), f"replay {t}"
        assert torch.equal(a.tokens, b.tokens) and torch.equal(a.lengths, b.lengths)
    assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)


@pytest.mark.parametrize("merge", [False, True])
def test_one_row_graph_replays_equal_eager_steps(small, merge):
    """The one-row step (norms in the residual epilogues, RoPE in the qkv epilogue; with `merge` the
    attention combine in the o projection) captured and replayed equals eager steps bit for bit."""
    model, _ = small
    print_case("graph replay one row", merge)
    try:
        model.fuse_attn_merge = merge
        a, b = model.new_state(1, 32), model.new_state(1, 32)
        tok = torch.tensor([321])
        a.set_tokens(tok, model.cfg.vocab_size)
        b.set_tokens(tok, model.cfg.vocab_size)
        graph = model.capture(b)
        for t in range(5):
            model.step(a)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(a.logits, b.logits), f"replay {t}"
            assert torch.equal(a.tokens, b.tokens) and torch.equal(a.lengths, b.lengths)
        assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)
    finally:
        model.fuse_attn_merge = False


def test_attn_merge_step_matches_reference_both_ways(small):
    """One row with the attention combine in the o projection and with the combine launch (the
    default): both within the reference bar of the step oracle (_run_and_compare)."""
    model, refs = small
    try:
        for flag in (True, False):
            model.fuse_attn_merge = flag
            _run_and_compare(model, refs, 1, steps=5, seed=23)
    finally:
        model.fuse_attn_merge = False


def test_one_row_step_with_1024_or_more_qkv_tiles():
    """A one-row step whose fused q|k|v projection has 1024 or more row tiles of 16 (MHA, 43 heads:
    129 heads of 128 rows = 1032 tiles) keeps the separate RoPE (the epilogue form takes fewer than
    1024 tiles): eager steps match the reference and graph replays equal them."""
    from scratch_llm_amd.decode import DecodeConfig, Int4DecodeLM

    print_case("one-row step, 1032 qkv tiles")
    dims = dict(vocab=512, d_model=43 * 128, n_layers=1, n_heads=43, n_kv_heads=43, d_ff=512)
    p = D.random_params(**dims, seed=5, std=0.02)
    cfg = DecodeConfig(vocab_size=dims["vocab"], d_model=dims["d_model"], n_layers=1, n_heads=43, n_kv_heads=43,
                       d_ff=dims["d_ff"], context_length=16)
    model = Int4DecodeLM.from_state_dict(cfg, lambda n: p[n], DEV)
    refs = {dt: D.int4_model(p, n_layers=1, n_heads=43, n_kv_heads=43, context_length=16, dtype=dt)
            for dt in (torch.bfloat16, torch.float32)}
    _run_and_compare(model, refs, 1, steps=3, seed=3, max_ctx=8)
    a, b = model.new_state(1, 8), model.new_state(1, 8)
    a.set_tokens(torch.tensor([7]), cfg.vocab_size)
    b.set_tokens(torch.tensor([7]), cfg.vocab_size)
    graph = model.capture(b)
    for t in range(3):
        model.step(a)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(a.logits, b.logits), f"replay {t}"


def test_inactive_slots_do_not_leak(small):
    """tests/test_batched_cache.py:186-213 on the device: garbage in inactive slots changes no bit of
    an active row, and advance leaves inactive rows where they were."""
    model, _ = small
    print_case("poisoned slots")
    a, b = model.new_state(4, 32), model.new_state(4, 32)
    for s in (a, b):
        s.active.copy_(torch.tensor([1, 0, 1, 0], dtype=torch.uint8))
        s.set_lengths([3, 9, 0, 31])
    b.k[:, 1].normal_()
    b.v[:, 3].normal_()
    tok = torch.tensor([1, 2, 3, 4])
    for _ in range(3):
        model.step(a, tok)
        model.step(b, tok)
        torch.cuda.synchronize()
        for r in (0, 2):
            assert torch.equal(a.logits[r], b.logits[r])
        tok = a.tokens.cpu()
    assert a.lengths.cpu().tolist() == [6, 9, 3, 31]


def test_step_rejects_bad_tokens(small):
    model, _ = small
    st = model.new_state(2, 16)
    with pytest.raises(IndexError):
        model.step(st, [0, model.cfg.vocab_size])
    with pytest.raises(ValueError):
        model.step(st, [0, 1, 2])


# ---------------------------------------------------------------------------------------------
# FP8 (per-head E4M3) KV cache
# ---------------------------------------------------------------------------------------------
def _valid_codes(shape, g):
    """Random E4M3 codes without the NaN encodings."""
    mag = torch.randint(0, 0x7F, shape, generator=g, dtype=torch.int32)
    sign = torch.randint(0, 2, shape, generator=g, dtype=torch.int32) << 7
    return (mag | sign).to(torch.uint8)


@pytest.mark.parametrize("H,Hkv,T", [(32, 8, 2048), (8, 8, 300), (16, 2, 77)])
def test_attention_fp8kv_brute_force(lib, H, Hkv, T):
    from oracle import fp8_ref as F8

    print_case("attention fp8 kv", H, Hkv, T)
    hd, B = 128, 4
    g = torch.Generator().manual_seed(H + T)
    lengths = [T - 1, 0, T // 3, T + 4]
    q = (torch.randn(B, H, hd, generator=g) * 2).bfloat16()
    kc, vc = _valid_codes((B, Hkv, T, hd), g), _valid_codes((B, Hkv, T, hd), g)
    ks = torch.rand(Hkv, generator=g) * 0.01 + 0.001
    vs = torch.rand(Hkv, generator=g) * 0.01 + 0.001
    out = torch.empty(B, H * hd, dtype=torch.bfloat16, device=DEV)
    nb = lib.sqx_attn_workspace_bytes(B, H, Hkv, T)
    ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
    ln = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    kd, vd, ksd, vsd = kc.to(DEV), vc.to(DEV), ks.to(DEV), vs.to(DEV)
    _ok(lib, lib.sqx_decode_attention_fp8kv(q.to(DEV).data_ptr(), kd.data_ptr(), vd.data_ptr(), ksd.data_ptr(),
                                            vsd.data_ptr(), ln.data_ptr(), B, H, Hkv, hd, T, out.data_ptr(),
                                            ws.data_ptr(), nb, _s()))
    torch.cuda.synchronize()
    kdeq = torch.from_numpy(F8.e4m3_decode(kc.numpy())).double() * ks.double().view(1, Hkv, 1, 1)
    vdeq = torch.from_numpy(F8.e4m3_decode(vc.numpy())).double() * vs.double().view(1, Hkv, 1, 1)
    G = H // Hkv
    got = out.cpu().view(B, H, hd).double()
    for b in range(B):
        L = min(max(lengths[b], 0) + 1, T)
        kk = kdeq[b, :, :L].repeat_interleave(G, dim=0)
        vv = vdeq[b, :, :L].repeat_interleave(G, dim=0)
        p = torch.softmax(torch.einsum("hd,htd->ht", q[b].double(), kk) / math.sqrt(hd), dim=-1)
        want = torch.einsum("ht,htd->hd", p, vv)
        bound = 2.0**-8 * want.abs() + 1e-5 * vv.abs().max()
        assert float(((got[b] - want).abs() / bound).max()) <= 1.0, f"row {b}"


@pytest.mark.parametrize("B,T", [(5, 300), (64, 2048)])
def test_fused_rope_fp8kv_equals_separate_steps(lib, B, T):
    """sqx_decode_attention_rope_fp8kv == (RoPE, quantize the new row with the head scales, then
    sqx_decode_attention_fp8kv), bit for bit: output and every cache byte."""
    from oracle import fp8_ref as F8

    print_case("fused rope fp8 kv", B, T)
    H, Hkv, hd, ctx = 32, 8, 128, T + 16
    g = torch.Generator().manual_seed(B + T)
    lengths = torch.randint(0, T, (B,), generator=g)
    lengths[0], lengths[1] = T - 1, 0
    lengths[2] = T + 3
    qkv = (torch.randn(B, (H + 2 * Hkv) * hd, generator=g) * 2).bfloat16()
    kc, vc = _valid_codes((B, Hkv, T, hd), g), _valid_codes((B, Hkv, T, hd), g)
    ks = torch.rand(Hkv, generator=g) * 0.02 + 0.002
    vs = torch.rand(Hkv, generator=g) * 0.02 + 0.002
    cos, sin = (t.to(DEV) for t in D.rope_tables(hd, ctx, 10000.0))
    ln = lengths.to(torch.int32).to(DEV)
    nb = lib.sqx_attn_workspace_bytes(B, H, Hkv, T)
    ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
    ksd, vsd = ks.to(DEV), vs.to(DEV)
    # fused
    k1, v1 = kc.to(DEV), vc.to(DEV)
    o1 = torch.empty(B, H * hd, dtype=torch.bfloat16, device=DEV)
    _ok(lib, lib.sqx_decode_attention_rope_fp8kv(qkv.to(DEV).data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                                 ctx, k1.data_ptr(), v1.data_ptr(), ksd.data_ptr(), vsd.data_ptr(), B, H,
                                                 Hkv, hd, T, o1.data_ptr(), ws.data_ptr(), nb, _s()))
    # separate: RoPE into bf16 scratch, quantize the new rows on the host oracle, attention on the codes
    q = torch.empty(B, H, hd, dtype=torch.bfloat16, device=DEV)
    kb = torch.zeros(B, Hkv, T, hd, dtype=torch.bfloat16, device=DEV)
    vb = torch.zeros_like(kb)
    _ok(lib, lib.sqx_rope_kv(qkv.to(DEV).data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx, B, H, Hkv, hd,
                             T, q.data_ptr(), kb.data_ptr(), vb.data_ptr(), _s()))
    torch.cuda.synchronize()
    k2, v2 = kc.clone(), vc.clone()
    slot = lengths.clamp(max=T - 1)
    for b in range(B):
        for src, dst, sc in ((kb, k2, ks), (vb, v2, vs)):
            row = src[b, :, int(slot[b])].float().cpu().numpy()  # [Hkv, hd]
            dst[b, :, int(slot[b])] = torch.from_numpy(
                F8.e4m3_encode_sat(row / sc.numpy()[:, None].astype(np.float32)))
    k2d, v2d = k2.to(DEV), v2.to(DEV)
    o2 = torch.empty_like(o1)
    _ok(lib, lib.sqx_decode_attention_fp8kv(q.data_ptr(), k2d.data_ptr(), v2d.data_ptr(), ksd.data_ptr(), vsd.data_ptr(),
                                            ln.data_ptr(), B, H, Hkv, hd, T, o2.data_ptr(), ws.data_ptr(), nb, _s()))
    torch.cuda.synchronize()
    assert torch.equal(k1.cpu(), k2) and torch.equal(v1.cpu(), v2)
    assert torch.equal(o1, o2)


def _fp8_scales(n_layers, hkv):
    return [torch.full((hkv,), 0.02) for _ in range(n_layers)], [torch.full((hkv,), 0.015) for _ in range(n_layers)]


@pytest.mark.parametrize("B", [1, 3])
def test_decode_step_fp8kv_matches_reference(small, B):
    model, refs = small
    print_case("decode step fp8 kv", B)
    cfg = model.cfg
    ks, vs = _fp8_scales(cfg.n_layers, cfg.n_kv_heads)
    st = model.new_state(B, 48, kv_dtype="fp8")
    for li in range(cfg.n_layers):
        st.set_kv_scales(li, ks[li].to(DEV), vs[li].to(DEV))
    caches = {dt: D.RefCache.empty(r, B, 48, dt, k_scale=ks, v_scale=vs) for dt, r in refs.items()}
    tok = torch.randint(0, cfg.vocab_size, (B,), generator=torch.Generator().manual_seed(B))
    for t in range(6):
        nxt = model.step(st, tok)
        torch.cuda.synchronize()
        got = st.logits.float().cpu()
        l16 = D.decode_step(refs[torch.bfloat16], caches[torch.bfloat16], tok, torch.bfloat16).float()
        l32 = D.decode_step(refs[torch.float32], caches[torch.float32], tok, torch.float32)
        scale = float(l32.abs().max())
        e_hip, e_ref = float((got - l32).abs().max()), float((l16 - l32).abs().max())
        assert e_hip <= 2 * e_ref + 2.0**-9 * scale, f"t={t}: {e_hip:.4g} vs {e_ref:.4g}"
        top2 = l32.topk(2, dim=-1).values
        sure = (top2[:, 0] - top2[:, 1]) > 4 * e_hip
        assert torch.equal(nxt.cpu().long()[sure], l32.argmax(-1)[sure])
        tok = nxt.cpu().long()
    assert st.k.dtype == torch.uint8 and st.k.element_size() == 1


def test_fp8kv_graph_replays_equal_eager(small):
    model, _ = small
    print_case("fp8 kv graph replay")
    cfg = model.cfg
    ks, vs = _fp8_scales(cfg.n_layers, cfg.n_kv_heads)
    a, b = model.new_state(4, 32, kv_dtype="fp8"), model.new_state(4, 32, kv_dtype="fp8")
    for s in (a, b):
        for li in range(cfg.n_layers):
            s.set_kv_scales(li, ks[li].to(DEV), vs[li].to(DEV))
        s.set_tokens(torch.tensor([5, 17, 300, 999]), cfg.vocab_size)
    graph = model.capture(b)
    for t in range(4):
        model.step(a)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(a.logits, b.logits), f"replay {t}"
    assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)
