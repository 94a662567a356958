"""The Llama block's elementwise kernels (add + RMSNorm, RoPE + head layout,
grouped-query attention without head copies) against the torch op sequences
they replace -- the HF Llama layer the reference wraps
(EE/python/dispatch.py:150-247) computes them with exactly these ops.

Bars: RoPE and the q/k/v layouts bit-exact (each op is one fp16-rounded
torch op); add + RMSNorm bit-exact in the residual sum; the normalised rows
equal torch's w * fp16(xf * r) with that fp16 intermediate at most one ulp
away (the f32 mean sums in another order than torch's reduction), >= 99% of
them bit-exact; the GQA attention within fp16 rounding
of the repeat_interleave form (the batched products change shape, so
hipBLASLt may pick another kernel and summation order).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ee():
    import entropy_engine
    return entropy_engine


def check_rmsnorm(n, s, w, eps, min_exact=0.99):
    """n == torch's w * fp16(xf * r), or the same with the fp16 intermediate one
    ulp away (a last-bit difference in the f32 mean), >= min_exact bit-exact."""
    xf = s.float()
    mid = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(torch.float16)
    ref = w * mid
    exact = n.view(torch.int16) == ref.view(torch.int16)
    assert exact.float().mean().item() >= min_exact
    up = torch.nextafter(mid, torch.full_like(mid, float("inf")))
    dn = torch.nextafter(mid, torch.full_like(mid, float("-inf")))
    ok = exact | (n.view(torch.int16) == (w * up).view(torch.int16)) | (n.view(torch.int16) == (w * dn).view(torch.int16))
    assert ok.all(), f"{(~ok).sum().item()} elements beyond a one-ulp intermediate"


@pytest.mark.parametrize("T,D", [(4096, 2048), (37, 256), (5, 4096), (1, 8), (64, 520)])
@pytest.mark.parametrize("residual", [False, True])
def test_add_rmsnorm(ee, T, D, residual):
    g = torch.Generator(device="cuda").manual_seed(T + D)
    x = torch.randn(T, D, device="cuda", generator=g).half() * 3
    y = torch.randn(T, D, device="cuda", generator=g).half() if residual else None
    w = (1 + 0.1 * torch.randn(D, device="cuda", generator=g)).half()
    s, n = ee.add_rmsnorm(x, w, 1e-5, y)
    s_ref = x + y if residual else x
    assert torch.equal(s, s_ref)
    check_rmsnorm(n, s_ref, w, 1e-5)


def test_add_rmsnorm_strided_and_errors(ee):
    x = torch.randn(16, 3 * 256, device="cuda").half()
    w = torch.ones(256, device="cuda", dtype=torch.float16)
    view = x[:, 256:512]                              # row stride 768
    _, n = ee.add_rmsnorm(view, w, 1e-6)
    check_rmsnorm(n, view, w, 1e-6)
    from entropy_engine import _lib
    with pytest.raises(_lib.EngineError):
        ee.add_rmsnorm(torch.zeros(4, 12, device="cuda", dtype=torch.float16),
                       torch.ones(12, device="cuda", dtype=torch.float16), 1e-6)


def torch_rope(x, cos, sin):
    h = x.shape[-1] // 2
    rot = torch.cat((-x[..., h:], x[..., :h]), dim=-1)
    return x * cos.unsqueeze(1) + rot * sin.unsqueeze(1)


def rope_tables(S, d, theta=10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, device="cuda", dtype=torch.float32) / d))
    f = torch.outer(torch.arange(S, device="cuda", dtype=torch.float32), inv)
    emb = torch.cat((f, f), dim=-1)
    return emb.cos().half().unsqueeze(0), emb.sin().half().unsqueeze(0)


@pytest.mark.parametrize("B,S,Hq,Hkv,d", [(8, 512, 32, 4, 64), (2, 33, 4, 2, 32), (1, 7, 2, 2, 128)])
def test_qkv_rope(ee, B, S, Hq, Hkv, d):
    g = torch.Generator(device="cuda").manual_seed(B * S + d)
    qkv = (torch.randn(B * S, (Hq + 2 * Hkv) * d, device="cuda", generator=g) * 2).half()
    cos, sin = rope_tables(S, d)
    q, k, v = ee.qkv_rope(qkv, cos, sin, B, S, Hq, Hkv, d, 1.0)
    qr = qkv[:, :Hq * d].reshape(B, S, Hq, d).transpose(1, 2)
    kr = qkv[:, Hq * d:(Hq + Hkv) * d].reshape(B, S, Hkv, d).transpose(1, 2)
    vr = qkv[:, (Hq + Hkv) * d:].reshape(B, S, Hkv, d).transpose(1, 2)
    assert torch.equal(q, torch_rope(qr, cos, sin))
    assert torch.equal(k, torch_rope(kr, cos, sin))
    assert torch.equal(v, vr.contiguous())
    # the folded attention scale: fp16(rope(q) * s)
    qs, _, _ = ee.qkv_rope(qkv, cos, sin, B, S, Hq, Hkv, d, d ** -0.5)
    assert torch.equal(qs, (torch_rope(qr, cos, sin).float() * d ** -0.5).half())


def test_gqa_attention_without_head_copies(ee):
    """_attention_entropy's grouped-query form against the repeat_interleave form
    (scores in fp32 on the same fp16 inputs) and against the fused kernel's entropy."""
    from entropy_engine.dispatch import _attention_entropy
    B, Hq, Hkv, S, d = 2, 8, 2, 128, 64
    g = torch.Generator(device="cuda").manual_seed(9)
    q = torch.randn(B, Hq, S, d, device="cuda", generator=g).half()
    k = torch.randn(B, Hkv, S, d, device="cuda", generator=g).half()
    v = torch.randn(B, Hkv, S, d, device="cuda", generator=g).half()
    out, H = _attention_entropy(q, k, v, d ** -0.5, causal=True)
    kr = k.repeat_interleave(Hq // Hkv, dim=1).float()
    vr = v.repeat_interleave(Hq // Hkv, dim=1).float()
    sc = (q.float() @ kr.transpose(-1, -2)) * d ** -0.5
    mask = torch.ones(S, S, device="cuda", dtype=torch.bool).tril()
    p = torch.softmax(sc.masked_fill(~mask, float("-inf")), dim=-1)
    ref = p @ vr
    assert (out.float() - ref).abs().max().item() <= 2e-2 * ref.abs().max().item()
    h_ref = -(p * torch.log(p.clamp_min(1e-30))).sum(-1)
    assert torch.allclose(H, h_ref, rtol=2e-3, atol=2e-3)
