"""The allocation-free decode attention (sqx_decode_attention_rope_noalloc) against the workspace form
it shares its kernels with (sqx_decode_attention_rope), through the C ABI: bit-identical outputs and
cache writes on two calls in a row, the second with a smaller input (the scratch array keeps the first
call's partials, which the second must not read), and a refusal, before any launch, of a shape whose
partials do not fit the fixed scratch."""

from __future__ import annotations

import pytest
import torch

from oracle import decode_ref as D
from tests.conftest import print_case

pytestmark = pytest.mark.gpu
DEV = "cuda"
SQX_E_SPACE = -3


@pytest.fixture(scope="module")
def lib():
    from scratch_llm_amd import _lib

    return _lib.load()


def _s():
    return torch.cuda.current_stream().cuda_stream


def _case(B, H, Hkv, T, seed):
    hd, ctx = 128, T + 16
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(0, T, (B,), generator=g)
    lengths[0] = T - 1
    if B > 1:
        lengths[1] = 0
    qkv = (torch.randn(B, (H + 2 * Hkv) * hd, generator=g) * 2).bfloat16().to(DEV)
    cache = torch.randn(2, B, Hkv, T, hd, generator=g).bfloat16().to(DEV)
    cos, sin = (t.to(DEV) for t in D.rope_tables(hd, ctx, 10000.0))
    return qkv, cache, cos, sin, ctx, lengths.to(torch.int32).to(DEV)


def _run(lib, B, H, Hkv, T, seed, noalloc):
    qkv, cache, cos, sin, ctx, ln = _case(B, H, Hkv, T, seed)
    kc, vc = cache[0].clone(), cache[1].clone()
    out = torch.empty(B, H * 128, dtype=torch.bfloat16, device=DEV)
    if noalloc:
        rc = lib.sqx_decode_attention_rope_noalloc(qkv.data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx,
                                                   kc.data_ptr(), vc.data_ptr(), B, H, Hkv, 128, T, out.data_ptr(), _s())
    else:
        nb = lib.sqx_attn_workspace_bytes(B, H, Hkv, T)
        ws = torch.empty(nb // 4, dtype=torch.float32, device=DEV)
        rc = lib.sqx_decode_attention_rope(qkv.data_ptr(), ln.data_ptr(), cos.data_ptr(), sin.data_ptr(), ctx,
                                           kc.data_ptr(), vc.data_ptr(), B, H, Hkv, 128, T, out.data_ptr(),
                                           ws.data_ptr(), nb, _s())
    assert rc == 0, lib.sqx_last_error().decode()
    torch.cuda.synchronize()
    return out, kc, vc


def test_noalloc_attention_equals_workspace_form(lib):
    # each call smaller than the one before; B = 64 takes one key chunk per row (no partials), the
    # others leave their partials in the scratch array
    for B, H, Hkv, T, seed in ((64, 32, 8, 2048, 1), (16, 32, 8, 2048, 3), (3, 32, 8, 300, 2)):
        print_case("noalloc attention", B, H, Hkv, T)
        want = _run(lib, B, H, Hkv, T, seed, noalloc=False)
        got = _run(lib, B, H, Hkv, T, seed, noalloc=True)
        for a, b, name in zip(got, want, ("out", "k cache", "v cache")):
            assert torch.equal(a, b), f"B={B} T={T}: {name} differs from the workspace form"


def test_noalloc_attention_refuses_oversized_shape(lib):
    B, H, Hkv, T = 1024, 32, 8, 4096  # one key chunk per row: B * H * 130 * 4 bytes of partials
    need = lib.sqx_attn_workspace_bytes(B, H, Hkv, T)
    assert need > 8 << 20
    dummy = torch.zeros(64, dtype=torch.float32, device=DEV)
    p = dummy.data_ptr()
    rc = lib.sqx_decode_attention_rope_noalloc(p, p, p, p, 4096, p, p, B, H, Hkv, 128, T, p, _s())
    assert rc == SQX_E_SPACE
    assert "scratch" in lib.sqx_last_error().decode()
