"""Pins the AWQ oracle (oracle/quant_ref.py) against the reference's recorded AWQ figures on its own
test layer, the golden search results written by the reference (tests/golden/reference_vectors.json),
and the closed-form identities of its tests. CPU only."""

from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import torch

from oracle import quant_ref as R

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.json"


def awq_layer(seed: int, n_tokens: int = 512):
    """The reference test's layer (tests/test_quant_awq.py:37-49): Linear[256, 512], 8 salient x12."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(256, 512, generator=g) * 0.02
    x = torch.randn(n_tokens, 512, generator=g)
    sal = torch.randperm(512, generator=g)[:8]
    x[:, sal] *= 12.0
    return w.numpy(), x.numpy(), sal.numpy()


def _recovery(w, x_calib, x_eval):
    y_ref = x_eval @ w.T
    qn, sn = R.quantize_groupwise_int4(w)
    m_n = R.mse(y_ref, x_eval @ R.dequantize_groupwise_int4(qn, sn).T)
    s, ratio, _ = R.search_awq_scale(w, x_calib)
    q, gs, _ = R.quantize_awq_int4(w, s)
    m_a = R.mse(y_ref, x_eval @ R.awq_dequantize(q, gs, s).T)
    return m_n, m_a, ratio


def test_recorded_awq_figures(known_answers):
    ka = known_answers["awq"]
    rec = []
    for seed in range(5):
        w, x, _ = awq_layer(seed)
        m_n, m_a, ratio = _recovery(w, x, x)
        rec.append(m_n / m_a)
        if seed == 0:
            assert abs(m_n - ka["recorded_seed0_mse_naive"]) < 5e-5
            assert abs(m_a - ka["recorded_seed0_mse_awq"]) < 5e-5
            assert ratio == ka["recorded_ratio"]
    assert abs(np.mean(rec) - ka["recorded_recovery_mean"]) < 0.01
    assert abs(min(rec) - ka["recorded_recovery_min"]) < 0.01
    w, x, _ = awq_layer(1)
    m_n, m_a, _ = _recovery(w, x[:256], x[256:])
    assert abs(m_n / m_a - ka["recorded_heldout"]) < 0.01


def test_search_matches_reference_golden():
    cases = json.loads(GOLDEN.read_text())["awq_search"]["cases"]
    for c in cases:
        w, x, _ = awq_layer(c["seed"])
        s, ratio, cm = R.search_awq_scale(w, x)
        assert ratio == c["ratio"]
        assert abs(cm - c["calib_mse"]) <= 1e-6 * c["calib_mse"]
        head = np.array([struct.unpack("<f", bytes.fromhex(h))[0] for h in c["chan_scale_head"]], np.float32)
        assert np.allclose(s[:16], head, rtol=2e-6, atol=0)


def test_alpha_zero_is_naive_and_linear_identity():
    w, x, _ = awq_layer(2)
    q0, gs0, _ = R.quantize_awq_int4(w, np.ones(512, np.float32))
    qn, sn = R.quantize_groupwise_int4(w)
    assert np.array_equal(q0, qn) and np.array_equal(gs0, sn)
    s = R.normalize_scale(R.act_scale(x) ** np.float32(0.25))
    q, gs, _ = R.quantize_awq_int4(w, s)
    w_eff = R.awq_dequantize(q, gs, s)
    xb = R.round_bf16(x[:4])
    assert np.array_equal(R.awq_linear(xb, q, gs, s), R.linear_f64(xb, R.round_bf16(w_eff)))
