"""Write tests/golden/reference_vectors.json from andreidhoang/scratch_llm's own quant functions.

Run in the build container only, where the reference checkout is mounted:

    PYTHONPATH=/root/reference/src python tests/golden/gen_reference_vectors.py

It covers only behaviour that no known answer, closed form or invariant pins:
- torch's fp32 log2 rounding inside the MXFP4 no-overflow scale (`_e8m0_no_overflow_scale`,
  nvfp4_mxfp4.py:162-174) and `quantize_e8m0` (:150-159) near powers of two and binade midpoints;
- `e2m1_round_to_code` (:85-98) where fp32 distances tie: inputs above 2**24, infinities, NaN, and
  exact midpoints;
- `search_awq_scale` (awq.py:122-151): the chosen alpha and calibration MSE, which depend on torch's
  reduction order.

Inputs and outputs are stored as data (fp32 bit patterns in hex). Nothing here runs on the GPU box,
and the tests read only the JSON.
"""

from __future__ import annotations

import json
import math
import struct
from pathlib import Path

import torch

from scratch_llm.quant import awq as A  # noqa: E402  (reference, build container only)
from scratch_llm.quant import nvfp4_mxfp4 as F  # noqa: E402

OUT = Path(__file__).resolve().parent / "reference_vectors.json"


def f2h(v: float) -> str:
    return struct.pack("<f", v).hex()


def bits_list(t: torch.Tensor) -> list[str]:
    return [f2h(float(v)) for v in t.reshape(-1).tolist()]


def from_bits(u: int) -> float:
    return struct.unpack("<f", struct.pack("<I", u))[0]


def main() -> None:
    torch.manual_seed(0)
    out: dict = {"_about": __doc__.strip().splitlines()[0], "torch": torch.__version__}

    # -- MXFP4 block scale at powers of two: amax/6 at 2^k * (1 + j ulp) and just below -----------
    amaxes = []
    for k in list(range(-40, 13)) + [-126, -125, 100, 120, 126]:
        for j in range(0, 9):
            t = math.ldexp(1.0 + j * 2.0**-23, k)
            amaxes.append(float(torch.tensor(t, dtype=torch.float32) * 6.0))
            t = math.ldexp(1.0 - j * 2.0**-24, k)
            amaxes.append(float(torch.tensor(t, dtype=torch.float32) * 6.0))
        amaxes.append(float(torch.tensor(math.ldexp(6.0, k), dtype=torch.float32).nextafter(torch.tensor(1e38))))
    amaxes = sorted(set(a for a in amaxes if math.isfinite(a) and a > 0))
    blocks = []
    for a in amaxes:
        # a block whose max is `a`, with a few smaller entries that land near E2M1 midpoints
        row = torch.zeros(32, dtype=torch.float32)
        row[0] = a
        row[1] = -a * 0.7
        row[2] = a * 0.2501
        row[3] = -a / 6.0 * 5.0
        row[4] = a / 6.0 * 0.25
        blocks.append(row)
    x = torch.stack(blocks)
    q = F.mxfp4_quantize(x, block=32)
    out["mxfp4_scale_edges"] = {  # blocks of 32: entries 5..31 are zero (code 0)
        "x_head": bits_list(x[:, :5]),
        "rows": len(blocks),
        "s_block": bits_list(q.s_block),
        "codes_head": q.codes[:, :5].reshape(-1).tolist(),
        "tail_codes_zero": bool((q.codes[:, 5:] == 0).all()),
    }

    # -- quantize_e8m0 at binade midpoints 2^(k+1/2) -----------------------------------------------
    vals = []
    for k in range(-30, 31):
        mid = torch.tensor(math.ldexp(math.sqrt(2.0), k), dtype=torch.float32)
        for j in range(-4, 5):
            u = struct.unpack("<I", struct.pack("<f", float(mid)))[0] + j
            vals.append(from_bits(u))
    v = torch.tensor(vals, dtype=torch.float32)
    out["e8m0_midpoints"] = {"v": bits_list(v), "out": bits_list(F.quantize_e8m0(v))}

    # -- e2m1 codes where fp32 distances tie or are non-finite --------------------------------------
    special = [0.0, -0.0, 0.25, -0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -5.0, 6.0, 6.0000005, 7.0, 1e4,
               2.0**23, 2.0**24, 2.0**24 + 2, 2.0**25, 2.0**25 + 4, 2.0**26, 3e7, 1e30, -1e30, 3.4e38,
               float("inf"), float("-inf"), float("nan"), 1e-45, -1e-45, 1.4e-39]
    for m in (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0):
        u = struct.unpack("<I", struct.pack("<f", m))[0]
        special += [from_bits(u - 1), from_bits(u + 1), -from_bits(u - 1), -from_bits(u + 1)]
    s = torch.tensor(special, dtype=torch.float32)
    out["e2m1_specials"] = {"x": bits_list(s), "codes": F.e2m1_round_to_code(s).tolist()}

    # -- quantize_e4m3 near binade edges and the subnormal boundary ---------------------------------
    ev = []
    for k in range(-12, 9):
        u = struct.unpack("<I", struct.pack("<f", math.ldexp(1.0, k)))[0]
        ev += [from_bits(u + j) for j in range(-3, 4)]
    ev += [447.0, 448.0, 449.0, 464.0, 480.0, 1e6, 0.0, 2.0**-10, 3 * 2.0**-11, 2.0**-9 * 1.5]
    e = torch.tensor(ev, dtype=torch.float32)
    out["e4m3_edges"] = {"v": bits_list(e), "out": bits_list(F.quantize_e4m3(e))}

    # -- small NVFP4 / MXFP4 tensors (seeded) --------------------------------------------------------
    g = torch.Generator().manual_seed(7)
    w = torch.randn(8, 96, generator=g) * 0.03
    w[3, 5] = 0.9  # an outlier block
    w[6, :32] = 0.0  # an all-zero block
    nq = F.nvfp4_quantize(w, block=16)
    out["nvfp4_small"] = {"shape": list(w.shape), "x": bits_list(w), "codes": nq.codes.reshape(-1).tolist(),
                          "s_block": bits_list(nq.s_block), "s_global": f2h(float(nq.s_global))}
    mq = F.mxfp4_quantize(w, block=32)
    out["mxfp4_small"] = {"shape": list(w.shape), "x": bits_list(w), "codes": mq.codes.reshape(-1).tolist(),
                          "s_block": bits_list(mq.s_block)}

    # -- AWQ search on the reference test's layer construction (tests/test_quant_awq.py:37-49) -------
    awq = []
    for seed in range(5):
        g = torch.Generator().manual_seed(seed)
        w = torch.randn(256, 512, generator=g) * 0.02
        x = torch.randn(512, 512, generator=g)
        sal = torch.randperm(512, generator=g)[:8]
        x[:, sal] *= 12.0
        r = A.search_awq_scale(w, x)
        awq.append({"seed": seed, "ratio": r.ratio, "calib_mse": r.calib_mse,
                    "chan_scale_head": bits_list(r.chan_scale[:16])})
    out["awq_search"] = {"construction": "w=randn(256,512)*0.02; x=randn(512,512); sal=randperm(512)[:8]; "
                                         "x[:,sal]*=12 (one torch.Generator, seed)", "cases": awq}

    OUT.write_text(json.dumps(out, indent=0) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
