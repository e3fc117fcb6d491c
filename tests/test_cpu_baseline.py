"""The timed CPU baseline (oracle.reference_cpu_forward: moe.cu's control flow, every
local expert dequantised to fp32 inside the call, then the per-expert loop) computes the
same output as the oracle's pinned expert path (expert_forward after routing, rounded
once to bf16), so bench.py's cpu_baseline times the right work.  Small case: two local
experts at full width (H = 7168, I = 2048), a few tokens routed into both of them by a
hot bias."""
import numpy as np
import torch

from conftest import oracle


def _case(T=5, seed=20260606):
    o = oracle()
    g = torch.Generator().manual_seed(seed)
    E = 2
    offset = 254                                  # local experts 254, 255: the last group
    logits = torch.randn(T, 256, generator=g)
    bias = torch.randn(256, generator=g) * 0.1
    bias[254:] += 3.0
    bias_bf16 = bias.to(torch.bfloat16)
    x = torch.randn(T, 7168, generator=g)
    amax = x.view(T, 56, 128).abs().amax(dim=2)
    sc = amax / 448.0
    hs = (x.view(T, 56, 128) / sc[:, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(T, 7168)

    def weights(rows, cols):
        w = torch.randn(E, rows, cols, generator=g) * 0.02
        b = w.view(E, rows // 128, 128, cols // 128, 128)
        s = b.abs().amax(dim=(2, 4)) / 448.0
        q = (b / s[:, :, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(E, rows, cols)
        return q, s.float()

    w1, s1 = weights(4096, 7168)
    w2, s2 = weights(7168, 2048)
    return o, (logits, bias_bf16, hs, sc.t().contiguous(), w1, s1, w2, s2, offset, 2.5)


def test_reference_cpu_forward_equals_the_pinned_expert_path():
    o, args = _case()
    T = args[0].shape[0]
    out = torch.empty(T, 7168, dtype=torch.bfloat16)
    o.reference_cpu_forward(*args, out)
    ids, w = o.route(args[0], args[1], args[9])
    assert ((ids == 254).any(axis=1) & (ids == 255).any(axis=1)).all()   # both experts used
    acc = o.expert_forward(args[2], args[3], args[4], args[5], args[6], args[7], ids, w, args[8])
    ref = acc.to(torch.bfloat16)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert float(acc.abs().max()) > 0.1           # the expert path did real work


def test_reference_cpu_forward_sees_a_planted_mistake():
    """A wrong routing factor changes the baseline's output: the comparison above is not
    vacuous."""
    o, args = _case()
    T = args[0].shape[0]
    out = torch.empty(T, 7168, dtype=torch.bfloat16)
    bad = list(args)
    bad[9] = 2.0
    o.reference_cpu_forward(*bad, out)
    ids, w = o.route(args[0], args[1], args[9])
    acc = o.expert_forward(args[2], args[3], args[4], args[5], args[6], args[7], ids, w, args[8])
    assert not torch.equal(out.view(torch.int16), acc.to(torch.bfloat16).view(torch.int16))
