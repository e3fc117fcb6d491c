"""GPU parity of the activation quantizer (moe_mi355_quantize_fp8_blockwise) against
the oracle restatement of kernel.cu:998-1062.  Codes and scales must match bit for bit:

* random rows of several magnitudes, bf16 and fp32 inputs, ragged shapes (1 row,
  odd row counts, 128 and 384 columns: partial passes of a wave);
* crafted blocks: all zero, NaN, +-inf, signed zeros, subnormals, constant blocks,
  one dominant element, values next to e4m3 rounding midpoints;
* full size (8192 x 7168 bf16): sampled rows against the oracle, and on every row the
  round trip |e4m3(q) * scale - x| <= 2^-4 |x| + 2^-10 scale;
* the operator run on the quantizer's output stays within the forward tolerance.
"""
import numpy as np
import pytest
import torch

from conftest import oracle, pkg
from gpu_common import compare_to_oracle, config_inputs, note, run_forward

pytestmark = pytest.mark.gpu


def _rows(rows, cols, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    mag = torch.logspace(-8, 4, rows).unsqueeze(1) * torch.rand(1, cols // 128, generator=g).repeat_interleave(128, 1)
    x = torch.randn(rows, cols, generator=g) * mag
    return x.to(dtype)


def _check(x_cpu: torch.Tensor):
    k = pkg("kernel")
    q, s = k.quantize_fp8_blockwise(x_cpu.cuda())
    torch.cuda.synchronize()
    rq, rs = oracle().quantize_fp8_blockwise(x_cpu)
    gq = q.view(torch.uint8).cpu().numpy()
    gs = s.cpu().numpy()
    assert gs.shape == rs.shape and gq.shape == rq.shape
    nbad_s = int((gs.view(np.uint32) != rs.view(np.uint32)).sum())
    nbad_q = int((gq != rq).sum())
    assert nbad_s == 0 and nbad_q == 0, (nbad_s, nbad_q)


@pytest.mark.parametrize("rows,cols,dtype", [(64, 7168, torch.bfloat16), (37, 7168, torch.float32),
                                             (1, 128, torch.bfloat16), (9, 384, torch.float32),
                                             (130, 1024, torch.bfloat16), (8, 7168, torch.float32)])
def test_quantize_matches_oracle(rows, cols, dtype):
    note(f"[gpu] quantize rows={rows} cols={cols} {dtype}")
    _check(_rows(rows, cols, rows * 7 + cols, dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quantize_special_values(dtype):
    note(f"[gpu] quantize special values {dtype}")
    o = oracle()
    x = torch.randn(16, 7168, generator=torch.Generator().manual_seed(3))
    x[0, :128] = 0.0
    x[1, 5] = float("nan")
    x[1, 200] = float("inf")
    x[2, 300] = float("-inf")
    x[3, :128] = -0.0
    x[3, 128:256] = 1e-40 if dtype == torch.float32 else 1e-39   # subnormal inputs
    x[4, :128] = 3.0
    x[5, 0] = 1e30
    tab = torch.from_numpy(o.e4m3_table()[:127].astype(np.float32))
    mids = (tab[:-1] + tab[1:]) / 2
    x[6, :126] = mids / 448.0 * 2.0           # block absmax 2 -> scale 2/448: x * inv near midpoints
    x[6, 126] = 2.0
    x[7, 128:128 + 127] = tab * 0.25          # exact codes, absmax 112
    _check(x.to(dtype))


def test_quantize_full_size_properties():
    T, H = 8192, 7168
    note(f"[gpu] quantize full size {T}x{H}")
    k = pkg("kernel")
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn(T, H, generator=g, device="cuda").to(torch.bfloat16)
    q, s = k.quantize_fp8_blockwise(x)
    torch.cuda.synchronize()
    srep = s.t().repeat_interleave(128, dim=1)
    deq = q.to(torch.float32) * srep
    xf = x.float()
    bound = 2.0 ** -4 * xf.abs() + 2.0 ** -10 * srep
    assert bool(((deq - xf).abs() <= bound * (1 + 1e-6)).all())
    rows = torch.randperm(T, generator=torch.Generator().manual_seed(4))[:192].sort().values
    rq, rs = oracle().quantize_fp8_blockwise(x[rows.cuda()].cpu())
    assert np.array_equal(q[rows.cuda()].view(torch.uint8).cpu().numpy(), rq)
    assert np.array_equal(s[:, rows.cuda()].cpu().numpy().view(np.uint32), rs.view(np.uint32))


def test_operator_on_quantizer_output():
    """The quantizer feeds the operator: bf16 hidden rows -> (q, scales) -> forward,
    checked against the fp32 oracle of the forward on the same (q, scales)."""
    note("[gpu] forward on quantizer output (config 1)")
    k = pkg("kernel")
    d0 = config_inputs(1)
    T = d0["routing_logits"].shape[0]
    xb = (torch.randn(T, 7168, generator=torch.Generator(device="cuda").manual_seed(21), device="cuda")
          ).to(torch.bfloat16)
    q, s = k.quantize_fp8_blockwise(xb)
    d = dict(d0)
    d["hidden_states"] = q
    d["hidden_states_scale"] = s
    out = run_forward(d)
    st = compare_to_oracle(d, out, list(range(T)))
    note(f"[gpu] forward on quantizer output: {st}")
    assert st["frac_within"] == 1.0, st
