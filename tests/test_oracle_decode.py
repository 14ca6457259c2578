"""Pins the decode-step oracle (oracle/decode_ref.py) on the CPU: the reference's own laws and named
values for the cached decode (tests/test_kv_cache.py, tests/test_batched_cache.py,
tests/test_model.py), closed forms and float64 brute force."""

from __future__ import annotations

import math

import torch

from oracle import decode_ref as D

CFG = dict(vocab=50, d_model=64, n_layers=2, n_heads=4, n_kv_heads=2, d_ff=96)


def _model(dtype=torch.float32, n_kv_heads=2, seed=0, group_size=32, params=None):
    cfg = dict(CFG, n_kv_heads=n_kv_heads)
    p = params if params is not None else D.random_params(**cfg, seed=seed, std=0.2)
    return D.int4_model(p, n_layers=cfg["n_layers"], n_heads=cfg["n_heads"], n_kv_heads=n_kv_heads,
                        context_length=32, group_size=group_size, dtype=dtype), p


def test_decode_steps_match_full_recompute():
    """The law of tests/test_kv_cache.py:34-51: each cached step equals the uncached forward."""
    m, _ = _model()
    ids = [3, 1, 4, 1, 5, 9, 2, 6]
    cache = D.RefCache.empty(m, 1, 16, torch.float32)
    for t in range(len(ids)):
        step = D.decode_step(m, cache, torch.tensor([ids[t]]), torch.float32)[0]
        full = D.full_forward(m, torch.tensor([ids[: t + 1]]), torch.float32)[0, -1]
        torch.testing.assert_close(step, full)
    assert cache.lengths.tolist() == [len(ids)]


def test_write_decode_lands_at_per_row_offsets():
    """Named values of tests/test_batched_cache.py:64-81."""
    m, _ = _model()
    m.n_kv_heads, m.head_dim, m.n_layers = 1, 4, 1
    cache = D.RefCache.empty(m, 2, 8, torch.float32)
    cache.lengths[0] = 3
    k_new = torch.arange(8, dtype=torch.float32).reshape(2, 1, 1, 4)
    cache.write_decode(0, k_new, -k_new)
    assert torch.equal(cache.k[0][0, 0, 3], torch.tensor([0.0, 1.0, 2.0, 3.0]))
    assert torch.equal(cache.k[0][1, 0, 0], torch.tensor([4.0, 5.0, 6.0, 7.0]))
    assert torch.equal(cache.v[0][0, 0, 3], -torch.tensor([0.0, 1.0, 2.0, 3.0]))
    assert cache.k[0][0, 0, 0].abs().sum() == 0
    # a full slot rewrites its last position (kv_cache.py:203, lengths clamped to max_ctx - 1)
    cache.lengths[1] = 8
    cache.write_decode(0, k_new + 10, k_new)
    assert torch.equal(cache.k[0][1, 0, 7], torch.tensor([14.0, 15.0, 16.0, 17.0]))


def test_advance_bumps_only_active_rows():
    """Named values of tests/test_batched_cache.py:91-103."""
    m, _ = _model()
    cache = D.RefCache.empty(m, 3, 8, torch.float32)
    cache.lengths[:] = torch.tensor([4, 2, 0])
    cache.active[:] = torch.tensor([True, False, True])
    cache.advance()
    assert cache.lengths.tolist() == [5, 2, 1]


def test_rope_score_depends_only_on_offset():
    """The law of tests/test_model.py:79-94, plus position 0 = identity and kept pair norms."""
    torch.manual_seed(0)
    cos, sin = D.rope_tables(16, 128, 10000.0)
    q, k = torch.randn(1, 1, 1, 16), torch.randn(1, 1, 1, 16)

    def score(i, j):
        return (D.rope(q, torch.tensor([i]), cos, sin) * D.rope(k, torch.tensor([j]), cos, sin)).sum().item()

    assert abs(score(5, 0) - score(20, 15)) < 1e-4
    assert abs(score(5, 0) - score(6, 0)) > 1e-4
    x = torch.randn(2, 3, 4, 16)
    assert torch.equal(D.rope(x, torch.zeros(4, dtype=torch.long), cos, sin), x)
    r = D.rope(x, torch.tensor([1, 7, 50, 127]), cos, sin)
    torch.testing.assert_close(r[..., 0::2] ** 2 + r[..., 1::2] ** 2, x[..., 0::2] ** 2 + x[..., 1::2] ** 2)
    # per-row positions equal the shared path row by row (tests/test_batched_cache.py:145-156)
    pos = torch.tensor([[5, 6, 7, 8], [0, 1, 2, 3]])
    out = D.rope(x[:2], pos, cos, sin)
    for b in range(2):
        assert torch.equal(out[b: b + 1], D.rope(x[b: b + 1], pos[b], cos, sin))


def test_attention_brute_force_and_single_key():
    torch.manual_seed(1)
    q, k, v = torch.randn(2, 3, 1, 8), torch.randn(2, 3, 6, 8), torch.randn(2, 3, 6, 8)
    mask = (torch.arange(6)[None] <= torch.tensor([2, 5])[:, None])[:, None, None, :]
    got = D.attention(q, k, v, mask).double()
    for b, L in ((0, 3), (1, 6)):
        for h in range(3):
            s = [sum(float(q[b, h, 0, i]) * float(k[b, h, j, i]) for i in range(8)) / math.sqrt(8) for j in range(L)]
            mx = max(s)
            e = [math.exp(x - mx) for x in s]
            want = [sum(e[j] * float(v[b, h, j, i]) for j in range(L)) / sum(e) for i in range(8)]
            assert max(abs(got[b, h, 0, i].item() - want[i]) for i in range(8)) < 1e-5
    one = (torch.arange(6)[None] <= torch.tensor([0, 0])[:, None])[:, None, None, :]
    assert torch.equal(D.attention(q, k, v, one), v[:, :, :1])


def test_gqa_equals_mha_on_repeated_kv_heads():
    """repeat_interleave semantics (model.py:315-318): query head h reads kv head h // G."""
    m_gqa, p = _model(n_kv_heads=2, seed=3)
    hd = CFG["d_model"] // CFG["n_heads"]
    p_mha = dict(p)
    for i in range(CFG["n_layers"]):
        for n in ("k_proj", "v_proj"):
            w = p[f"blocks.{i}.attn.{n}.weight"].view(2, hd, -1)
            p_mha[f"blocks.{i}.attn.{n}.weight"] = w.repeat_interleave(2, dim=0).reshape(4 * hd, -1)
    m_mha, _ = _model(n_kv_heads=4, params=p_mha)
    c1 = D.RefCache.empty(m_gqa, 2, 8, torch.float32)
    c2 = D.RefCache.empty(m_mha, 2, 8, torch.float32)
    for tok in ([1, 2], [3, 4], [5, 6]):
        a = D.decode_step(m_gqa, c1, torch.tensor(tok), torch.float32)
        b = D.decode_step(m_mha, c2, torch.tensor(tok), torch.float32)
        torch.testing.assert_close(a, b)


def test_rmsnorm_closed_form():
    d, eps = 64, 1e-5
    w = 1.0 + 0.1 * torch.randn(d, generator=torch.Generator().manual_seed(4))
    for c in (0.0, 1e-3, 0.5, -3.0, 100.0):
        y = D.rmsnorm(torch.full((2, d), c), w, eps)
        want = (c / math.sqrt(c * c + eps)) * w.double()
        assert torch.allclose(y.double(), want.expand(2, d), rtol=1e-6, atol=1e-7)


def test_rows_do_not_leak_from_inactive_slots():
    """tests/test_batched_cache.py:186-213: active rows are bit-identical whatever inactive slots hold."""
    for dtype in (torch.float32, torch.bfloat16):
        m, _ = _model(dtype=dtype, seed=5)
        caches = [D.RefCache.empty(m, 3, 8, dtype) for _ in range(2)]
        for c in caches:
            c.active[:] = torch.tensor([True, False, True])
        g = torch.Generator().manual_seed(9)
        for layer in range(m.n_layers):
            caches[1].k[layer][1].normal_(generator=g)
            caches[1].v[layer][1].normal_(generator=g)
        for tok in ([1, 0, 2], [3, 0, 4]):
            a = D.decode_step(m, caches[0], torch.tensor(tok), dtype)
            b = D.decode_step(m, caches[1], torch.tensor(tok), dtype)
            for r in (0, 2):
                assert torch.equal(a[r], b[r])
        assert caches[0].lengths.tolist() == [2, 0, 2]


def test_bf16_composition_stays_near_fp32():
    """The bf16 composition and the fp32 run of the same parameters agree to bf16 precision."""
    p = D.random_params(**CFG, seed=6, std=0.2)
    m16, _ = _model(dtype=torch.bfloat16, params=p)
    m32, _ = _model(dtype=torch.float32, params=p)
    c16 = D.RefCache.empty(m16, 2, 8, torch.bfloat16)
    c32 = D.RefCache.empty(m32, 2, 8, torch.float32)
    for tok in ([1, 2], [3, 4], [5, 6]):
        a = D.decode_step(m16, c16, torch.tensor(tok), torch.bfloat16).float()
        b = D.decode_step(m32, c32, torch.tensor(tok), torch.float32)
        assert float((a - b).abs().max() / b.abs().max()) < 5e-2


def test_fp8_cache_write_is_the_fp8_oracles_round_trip():
    """The FP8 slot cache stores exactly dequantize_per_head(quantize_per_head(x, s), s)."""
    import numpy as np

    from oracle import fp8_ref as F8

    g = torch.Generator().manual_seed(12)
    k = torch.randn(3, 2, 1, 16, generator=g) * 5
    s = torch.tensor([0.01, 0.002])
    m, _ = _model()
    m.n_kv_heads, m.head_dim, m.n_layers = 2, 16, 1
    cache = D.RefCache.empty(m, 3, 4, torch.float32, k_scale=[s], v_scale=[s])
    cache.write_decode(0, k, k)
    want = F8.dequantize_per_head(F8.quantize_per_head(k.numpy(), s.view(1, 2, 1, 1).numpy()),
                                  s.view(1, 2, 1, 1).numpy())
    assert np.array_equal(cache.k[0][:, :, 0].numpy(), want[:, :, 0])
    ceiling = float(torch.tensor(448.0) * s[0])  # the fp32 product the dequantization forms
    assert float(cache.k[0][:, 0, 0].abs().max()) == ceiling  # saturated values land on the head's ceiling
