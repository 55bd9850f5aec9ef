"""GPU parity of the decoder-block kernels: attention, RMSNorm, RoPE, SwiGLU backward.

Every reference is float64 on the CPU over the same bf16/fp32 inputs; the
tolerances are error bounds built from the reference quantities: bf16
rounding is 2^-8 relative, fp32 accumulation is at most K 2^-23 of the sum of
magnitudes. Gradients are checked against float64 autograd.
"""

from __future__ import annotations

import math
import os
import sys

import pytest
import torch

from mround_amd import kernels as K
from tests.helpers import dev

pytestmark = pytest.mark.gpu

U = 2.0**-8  # bf16 unit roundoff


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------ attention --

def attention_ref(qkv, B, S, Hq, Hkv, D, scale, dout=None):
    """float64 causal GQA attention over packed [B*S, ld] rows; returns the
    output, the natural log-sum-exp, and (with dout) the gradient of the packed rows."""
    width = (Hq + 2 * Hkv) * D
    x = qkv[:, :width].double().clone().requires_grad_(dout is not None)
    t = x.reshape(B, S, Hq + 2 * Hkv, D)
    q = t[:, :, :Hq].permute(0, 2, 1, 3)
    k = t[:, :, Hq:Hq + Hkv].permute(0, 2, 1, 3).repeat_interleave(Hq // Hkv, 1)
    v = t[:, :, Hq + Hkv:].permute(0, 2, 1, 3).repeat_interleave(Hq // Hkv, 1)
    s = (q @ k.transpose(-1, -2)) * scale
    causal = torch.ones(S, S, dtype=torch.bool).tril()
    s = s.masked_fill(~causal, float("-inf"))
    lse = torch.logsumexp(s, -1)
    p = torch.exp(s - lse[..., None])
    o = p @ v  # [B, Hq, S, D]
    out = o.permute(0, 2, 1, 3).reshape(B * S, Hq * D)
    res = {"out": out.detach(), "lse": lse.detach(), "p": p.detach(), "q": q.detach(),
           "k": k.detach(), "v": v.detach()}
    if dout is not None:
        (out * dout.double()).sum().backward()
        res["dqkv"] = x.grad
    return res


ATTN_CASES = [
    # B, S, Hq, Hkv, D, magnitude
    (1, 128, 2, 1, 64, 1.0),
    (2, 256, 4, 2, 128, 1.0),
    (1, 384, 4, 4, 64, 1.0),
    (1, 256, 8, 1, 128, 1.0),
    (1, 512, 2, 2, 128, 3.0),
    (2, 128, 14, 2, 64, 2.0),
]


def _attn_inputs(B, S, Hq, Hkv, D, mag, seed, pad):
    width = (Hq + 2 * Hkv) * D
    ld = width + pad
    qkv = torch.full((B * S, ld), 7.0).to(torch.bfloat16)
    qkv[:, :width] = (torch.randn(B * S, width, generator=_gen(seed)) * mag).to(torch.bfloat16)
    return qkv, ld


@pytest.mark.parametrize("case", ATTN_CASES)
def test_attention_forward(case):
    B, S, Hq, Hkv, D, mag = case
    print("case attn fwd", case, flush=True, file=sys.stderr)
    qkv, _ = _attn_inputs(B, S, Hq, Hkv, D, mag, seed=21, pad=64)
    scale = 1.0 / math.sqrt(D)
    ref = attention_ref(qkv, B, S, Hq, Hkv, D, scale)
    ldo = Hq * D + 8
    out = torch.full((B * S, ldo), 5.0, dtype=torch.bfloat16, device=dev())
    lse = torch.empty(B, Hq, S, device=dev())
    K.attn_fwd(qkv.to(dev()), batch=B, seq_len=S, n_heads=Hq, n_kv_heads=Hkv, head_dim=D,
               scale=scale, out=out, lse=lse)
    got = out.double().cpu()
    assert torch.all(got[:, Hq * D:] == 5.0), "padding columns were written"
    o_ref = ref["out"]
    # P rounded to bf16 before P V, then one rounding of the output
    pv = (ref["p"] @ ref["v"].abs()).permute(0, 2, 1, 3).reshape(B * S, Hq * D)
    tol = 1.5 * U * pv + U * o_ref.abs() + 1e-6
    err = (got[:, :Hq * D] - o_ref).abs()
    print("  out max err/tol", float((err / tol).max()), file=sys.stderr)
    assert torch.all(err <= tol)
    assert torch.allclose(lse.double().cpu(), ref["lse"], rtol=0, atol=2e-5)


def _check_attention_backward(qkv, dout, got, B, S, Hq, Hkv, D, scale):
    """dQ, dK, dV of the kernel (``got``: float64 [B*S, (Hq + 2 Hkv) D]) against
    float64 autograd over the same bf16 inputs, within bounds built from the
    reference quantities (the kernel's own output, P and dS rounded to bf16)."""
    ref = attention_ref(qkv, B, S, Hq, Hkv, D, scale, dout=dout)
    got = got.reshape(B, S, Hq + 2 * Hkv, D)
    want = ref["dqkv"].reshape(B, S, Hq + 2 * Hkv, D)
    p, q, k, v = ref["p"], ref["q"], ref["k"], ref["v"]
    do = dout.double().reshape(B, S, Hq, D).permute(0, 2, 1, 3)
    o = ref["out"].reshape(B, S, Hq, D).permute(0, 2, 1, 3)
    dp = do @ v.transpose(-1, -2)
    ds = p * (dp - (do * o).sum(-1, keepdim=True))
    tol_o = 1.5 * U * (p @ v.abs()) + U * o.abs() + 1e-6  # the kernel's own output
    e_d = (do.abs() * tol_o).sum(-1, keepdim=True)
    e_ds = p * (e_d + 1e-6 * (do.abs() @ v.abs().transpose(-1, -2))) + 2 * U * ds.abs()
    G = Hq // Hkv

    def per_kv(x):  # sum the query heads of each group: [B, Hq, S, D] -> [B, Hkv, S, D]
        return x.reshape(B, Hkv, G, S, D).sum(2)

    tol_dq = scale * (e_ds @ k.abs()) * 1.5
    tol_dk = per_kv(scale * (e_ds.transpose(-1, -2) @ q.abs())) * 1.5
    tol_dv = per_kv(1.5 * U * (p.transpose(-1, -2) @ do.abs())) * 1.5
    for name, sl, tol in (("dq", slice(0, Hq), tol_dq), ("dk", slice(Hq, Hq + Hkv), tol_dk),
                          ("dv", slice(Hq + Hkv, Hq + 2 * Hkv), tol_dv)):
        w = want[:, :, sl].permute(0, 2, 1, 3)
        g = got[:, :, sl].permute(0, 2, 1, 3)
        t = tol + U * w.abs() + 1e-6
        err = (g - w).abs()
        print(f"  {name} max err/tol", float((err / t).max()), file=sys.stderr)
        assert torch.all(err <= t), name


def _run_attention(qkv, B, S, Hq, Hkv, D, dout, ld, *, hsplit=0):
    """Forward then backward on the GPU; returns dqkv (device, [B*S, ld], its
    padding columns pre-filled with 3.0)."""
    scale = 1.0 / math.sqrt(D)
    q_d = qkv.to(dev())
    out = torch.empty(B * S, Hq * D, dtype=torch.bfloat16, device=dev())
    lse = torch.empty(B, Hq, S, device=dev())
    K.attn_fwd(q_d, batch=B, seq_len=S, n_heads=Hq, n_kv_heads=Hkv, head_dim=D, scale=scale,
               out=out, lse=lse)
    dsum = torch.empty(B, Hq, S, device=dev())
    dqkv = torch.full((B * S, ld), 3.0, dtype=torch.bfloat16, device=dev())
    K.attn_bwd(q_d, out, dout.to(dev()), lse, dsum, batch=B, seq_len=S, n_heads=Hq, n_kv_heads=Hkv,
               head_dim=D, scale=scale, dqkv=dqkv, hsplit=hsplit)
    return dqkv


@pytest.mark.parametrize("case", ATTN_CASES)
def test_attention_backward(case):
    B, S, Hq, Hkv, D, mag = case
    print("case attn bwd", case, flush=True, file=sys.stderr)
    qkv, ld = _attn_inputs(B, S, Hq, Hkv, D, mag, seed=22, pad=32)
    width = (Hq + 2 * Hkv) * D
    dout = torch.randn(B * S, Hq * D, generator=_gen(23)).to(torch.bfloat16)
    got = _run_attention(qkv, B, S, Hq, Hkv, D, dout, ld).double().cpu()
    assert torch.all(got[:, width:] == 3.0), "padding columns were written"
    _check_attention_backward(qkv, dout, got[:, :width], B, S, Hq, Hkv, D, 1.0 / math.sqrt(D))


# Every way the dK/dV kernel can walk a group of G query heads: one block per
# kv head walking all G (hsplit 1, bf16 written directly: the Qwen2.5-7B
# launch, G = 7), uneven splits into fp32 partials (G = 7 over 2 blocks: 3 + 4
# heads, the Qwen2.5-0.5B launch; over 3: 2 + 2 + 3; G = 8 over 2: the
# Qwen2.5-3B launch) and one head per block (hsplit G).
SPLIT_CASES = [
    # B, S, Hq, Hkv, D, hsplit
    (1, 256, 14, 2, 64, 1), (1, 256, 14, 2, 64, 2), (1, 256, 14, 2, 64, 3), (1, 256, 14, 2, 64, 7),
    (2, 128, 14, 2, 128, 1), (2, 128, 14, 2, 128, 2), (2, 128, 14, 2, 128, 7),
    (1, 256, 8, 1, 128, 1), (1, 256, 8, 1, 128, 2), (1, 256, 8, 1, 128, 3), (1, 256, 8, 1, 128, 8),
    (1, 256, 16, 2, 64, 1), (1, 256, 16, 2, 64, 2), (1, 256, 16, 2, 64, 8),
]


@pytest.mark.parametrize("case", SPLIT_CASES)
def test_attention_backward_head_split(case):
    B, S, Hq, Hkv, D, hsplit = case
    print("case attn bwd split", case, flush=True, file=sys.stderr)
    qkv, ld = _attn_inputs(B, S, Hq, Hkv, D, 1.5, seed=24, pad=32)
    width = (Hq + 2 * Hkv) * D
    dout = torch.randn(B * S, Hq * D, generator=_gen(25)).to(torch.bfloat16)
    got = _run_attention(qkv, B, S, Hq, Hkv, D, dout, ld, hsplit=hsplit).double().cpu()
    assert torch.all(got[:, width:] == 3.0), "padding columns were written"
    _check_attention_backward(qkv, dout, got[:, :width], B, S, Hq, Hkv, D, 1.0 / math.sqrt(D))


class _PairKernel:
    """Every dK/dV launch at D = 128 inside the block runs on the two-waves-per-SIMD pair kernel."""

    def __enter__(self):
        os.environ["MR_ATTN_PAIR"] = "1"

    def __exit__(self, *exc):
        del os.environ["MR_ATTN_PAIR"]


# The pipelined dK/dV kernel (D = 128) against the pair kernel, bit for bit:
# both sum the same products in the same order. Item counts (32-query tiles
# times query heads per block) end at both positions of its 8-stage round
# (n mod 8 = 0, 4), with one and several heads per block, bf16 written
# directly and fp32 partials (hsplit > 1), and the 7B launch.
PIPE_CASES = [
    # B, S, Hq, Hkv, D, hsplit
    (1, 128, 2, 1, 128, 1), (1, 128, 3, 3, 128, 1), (2, 384, 14, 2, 128, 1), (2, 384, 14, 2, 128, 2),
    (1, 256, 8, 1, 128, 3), (1, 256, 8, 1, 128, 8), (8, 2048, 28, 4, 128, 0),
]


@pytest.mark.parametrize("case", PIPE_CASES)
def test_attention_dkdv_pipeline_matches_pair(case):
    B, S, Hq, Hkv, D, hsplit = case
    print("case attn bwd pipe vs pair", case, flush=True, file=sys.stderr)
    qkv, ld = _attn_inputs(B, S, Hq, Hkv, D, 1.5, seed=30, pad=16)
    dout = torch.randn(B * S, Hq * D, generator=_gen(31)).to(torch.bfloat16)
    got = _run_attention(qkv, B, S, Hq, Hkv, D, dout, ld, hsplit=hsplit)
    with _PairKernel():
        ref = _run_attention(qkv, B, S, Hq, Hkv, D, dout, ld, hsplit=hsplit)
    assert torch.equal(got, ref), "pipelined and pair dK/dV kernels differ"


class _DotFirst:
    """Attention backward launches inside the block form D = rowsum(dO O) with
    the separate attn_bwd_dot kernel first and run dQ last."""

    def __enter__(self):
        os.environ["MR_ATTN_DOT"] = "1"

    def __exit__(self, *exc):
        del os.environ["MR_ATTN_DOT"]


@pytest.mark.parametrize("case", PIPE_CASES + [(2, 256, 4, 2, 64, 1), (1, 384, 8, 2, 64, 2)])
def test_attention_dq_forms_the_row_sums(case):
    # The dQ kernel forms D itself (the dot kernel's products and sums in the
    # same order), writes it for the dK/dV kernel and runs first: dQ, dK and
    # dV bit-identical to the separate dot kernel's order, at D = 64 and 128,
    # with head splits, and the 7B launch.
    B, S, Hq, Hkv, D, hsplit = case
    print("case attn bwd row sums in dQ", case, flush=True, file=sys.stderr)
    qkv, ld = _attn_inputs(B, S, Hq, Hkv, D, 1.5, seed=34, pad=16)
    dout = torch.randn(B * S, Hq * D, generator=_gen(35)).to(torch.bfloat16)
    got = _run_attention(qkv, B, S, Hq, Hkv, D, dout, ld, hsplit=hsplit)
    with _DotFirst():
        ref = _run_attention(qkv, B, S, Hq, Hkv, D, dout, ld, hsplit=hsplit)
    assert torch.equal(got, ref), "the row sums formed in dQ differ from the dot kernel's"


def test_attention_head_splits_agree():
    """The split changes only the order dK/dV partials are summed in: every
    split of one problem agrees within a few bf16 units (dQ is bit-identical)."""
    B, S, Hq, Hkv, D = 1, 256, 14, 2, 64
    qkv, ld = _attn_inputs(B, S, Hq, Hkv, D, 1.5, seed=26, pad=0)
    dout = torch.randn(B * S, Hq * D, generator=_gen(27)).to(torch.bfloat16)
    runs = {h: _run_attention(qkv, B, S, Hq, Hkv, D, dout, ld, hsplit=h).float().cpu() for h in (1, 2, 7)}
    for h in (2, 7):
        assert torch.equal(runs[h][:, :Hq * D], runs[1][:, :Hq * D]), "dQ depends on the split"
        kv = slice(Hq * D, None)
        assert torch.allclose(runs[h][:, kv], runs[1][:, kv], rtol=4 * U, atol=1e-3)


@pytest.mark.parametrize("hsplit", [0, 2])
def test_attention_backward_7b_launch(hsplit):
    """The exact launch of the Qwen2.5-7B block tune (8 x 2048 tokens, 28 query
    and 4 kv heads of 128: 512 dK/dV blocks, each walking its group's 7 query
    heads; hsplit 0 is the automatic choice, 1 there) and the same over fp32
    partials, checked on one (sequence, kv head) slice against float64."""
    B, S, Hq, Hkv, D = 8, 2048, 28, 4, 128
    print("case attn bwd 7b", hsplit, flush=True, file=sys.stderr)
    assert K.attn_bwd_workspace_bytes(batch=B, seq_len=S, n_heads=Hq, n_kv_heads=Hkv, head_dim=D) == 0
    qkv, ld = _attn_inputs(B, S, Hq, Hkv, D, 1.0, seed=28, pad=0)
    dout = torch.randn(B * S, Hq * D, generator=_gen(29)).to(torch.bfloat16)
    got = _run_attention(qkv, B, S, Hq, Hkv, D, dout, ld, hsplit=hsplit).cpu()
    G, b, g = Hq // Hkv, 5, 2
    rows = slice(b * S, (b + 1) * S)
    cols = list(range(g * G * D, (g + 1) * G * D)) + list(range((Hq + g) * D, (Hq + g + 1) * D)) + \
        list(range((Hq + Hkv + g) * D, (Hq + Hkv + g + 1) * D))
    _check_attention_backward(qkv[rows][:, cols], dout[rows][:, g * G * D:(g + 1) * G * D],
                              got[rows][:, cols].double(), 1, S, G, 1, D, 1.0 / math.sqrt(D))


def test_attention_rejects_bad_shapes():
    qkv = torch.zeros(200, 4 * 64, dtype=torch.bfloat16, device=dev())
    out = torch.zeros(200, 2 * 64, dtype=torch.bfloat16, device=dev())
    lse = torch.zeros(200 * 2, device=dev())
    with pytest.raises(Exception, match="multiple of 128"):
        K.attn_fwd(qkv, batch=1, seq_len=200, n_heads=2, n_kv_heads=1, head_dim=64, scale=0.125,
                   out=out, lse=lse)
    with pytest.raises(Exception, match="head_dim"):
        K.attn_fwd(qkv[:128], batch=1, seq_len=128, n_heads=1, n_kv_heads=1, head_dim=96,
                   scale=0.125, out=out[:128], lse=lse)


# ------------------------------------------------------------------- RMSNorm --

def rmsnorm_ref(h, w, eps):
    h64 = h.double()
    r = 1.0 / torch.sqrt((h64 * h64).mean(-1, keepdim=True) + eps)
    return h64 * r * w.double(), r


# rows of width % 4 == 0 take the vectorized kernels (row held in registers);
# 130 and 9 take the scalar ones
@pytest.mark.parametrize("shape", [(300, 896), (64, 3584), (8, 128), (17, 4096), (5, 130), (3, 9)])
def test_rmsnorm_forward(shape):
    T, H = shape
    h = torch.randn(T, H, generator=_gen(31)) * 3
    w = 1 + 0.1 * torch.randn(H, generator=_gen(32))
    y_ref, r_ref = rmsnorm_ref(h, w, 1e-6)
    y = torch.empty(T, H, dtype=torch.bfloat16, device=dev())
    rstd = torch.empty(T, device=dev())
    K.rmsnorm_fwd(h.to(dev()), w.to(dev()), 1e-6, y, rstd)
    tol = U * y_ref.abs() * (1 + 1e-5) + 1e-5 * y_ref.abs() + 1e-30
    assert torch.all((y.double().cpu() - y_ref).abs() <= tol)
    assert torch.allclose(rstd.double().cpu(), r_ref[:, 0], rtol=1e-5, atol=0)


@pytest.mark.parametrize("shape", [(300, 896), (64, 3584), (7, 130)])
@pytest.mark.parametrize("with_res", [False, True])
def test_rmsnorm_backward(shape, with_res):
    T, H = shape
    h = torch.randn(T, H, generator=_gen(33)) * 2
    w = 1 + 0.1 * torch.randn(H, generator=_gen(34))
    dy = torch.randn(T, H, generator=_gen(35))
    dres = torch.randn(T, H, generator=_gen(36)) if with_res else None
    h64 = h.double().requires_grad_(True)
    y64, r64 = rmsnorm_ref(h64, w, 1e-6)
    (y64 * dy.double()).sum().backward()
    want = h64.grad + (dres.double() if with_res else 0)
    r = r64.detach()
    mags = (r * (w.double() * dy.double()).abs()
            + r**3 * h.double().abs() / H * (dy.double() * w.double() * h.double()).abs().sum(-1, keepdim=True))
    if with_res:
        mags = mags + dres.double().abs()
    hd, wd, dyd = h.to(dev()), w.to(dev()), dy.to(dev())
    rstd = torch.empty(T, device=dev())
    K.rmsnorm_fwd(hd, wd, 1e-6, torch.empty(T, H, dtype=torch.bfloat16, device=dev()), rstd)
    dh32 = torch.empty(T, H, device=dev())
    dh16 = torch.empty(T, H, dtype=torch.bfloat16, device=dev())
    K.rmsnorm_bwd(dyd, hd, wd, rstd, dres.to(dev()) if with_res else None, dh_bf16=dh16, dh_f32=dh32)
    tol = 2e-5 * mags + 1e-30
    assert torch.all((dh32.double().cpu() - want).abs() <= tol)
    assert torch.all((dh16.double().cpu() - want).abs() <= tol + U * want.abs())


# ---------------------------------------------------------------------- RoPE --

def rope_table(S, d, base=10000.0):
    inv = 1.0 / (base ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    ang = torch.arange(S, dtype=torch.float64)[:, None] * inv[None, :]
    return torch.stack([torch.cos(ang), torch.sin(ang)], -1).float()  # [S, d/2, 2]


def rope_ref(x, S, n_heads, d, cs, backward):
    """float64 rotation of the first n_heads heads of each row (halves layout)."""
    T = x.shape[0]
    y = x.double().clone()
    pos = torch.arange(T) % S
    c = cs[pos, :, 0].double()[:, None, :]
    s = cs[pos, :, 1].double()[:, None, :]
    if backward:
        s = -s
    h = y[:, :n_heads * d].reshape(T, n_heads, d)
    a, b = h[..., :d // 2].clone(), h[..., d // 2:].clone()
    h[..., :d // 2] = a * c - b * s
    h[..., d // 2:] = b * c + a * s
    y[:, :n_heads * d] = h.reshape(T, n_heads * d)
    mag = torch.zeros_like(y)
    m = (a.abs() * c.abs() + b.abs() * s.abs())
    mag[:, :n_heads * d] = torch.cat([m, m], -1).reshape(T, n_heads * d)
    return y, mag


# head_dim % 16 == 0 with 16-byte rows takes the 8-pair kernel; 40 the scalar one
@pytest.mark.parametrize("cfg", [(2, 128, 6, 2, 64), (1, 256, 16, 4, 128), (3, 40, 2, 1, 128),
                                 (2, 24, 3, 1, 40)])
@pytest.mark.parametrize("backward", [False, True])
def test_rope(cfg, backward):
    B, S, Hq, Hkv, d = cfg
    T = B * S
    width = (Hq + 2 * Hkv) * d
    x = torch.randn(T, width + 16, generator=_gen(41)).to(torch.bfloat16)
    cs = rope_table(S, d, base=1e6)
    y_ref, mag = rope_ref(x, S, Hq + Hkv, d, cs, backward)
    xd = x.to(dev())
    K.rope(xd, seq_len=S, n_heads=Hq + Hkv, head_dim=d, cos_sin=cs.to(dev()), backward=backward)
    got = xd.double().cpu()
    tol = U * y_ref.abs() + 4 * 2.0**-24 * mag
    assert torch.all((got - y_ref).abs() <= tol)
    # v heads and padding untouched
    assert torch.equal(got[:, (Hq + Hkv) * d:], x.double()[:, (Hq + Hkv) * d:])


# ---------------------------------------------------------------------- cast --

@pytest.mark.parametrize("n,offset", [(4096, 0), (1000, 0), (1001, 0), (1000, 1)])
def test_cast_bf16(n, offset):
    """fp32 -> bf16, round to nearest even (vectorized when n % 4 == 0 and aligned)."""
    x = torch.randn(n + offset, generator=_gen(47)) * 100
    x[offset + 3] = 1.0 + 2.0 ** -8  # a tie: rounds to even (1.0)
    xd = x.to(dev())[offset:]
    y = torch.empty(n + offset, dtype=torch.bfloat16, device=dev())[offset:]
    K.cast_bf16(xd, y)
    assert torch.equal(y.cpu(), x[offset:].to(torch.bfloat16))


# -------------------------------------------------------------- SwiGLU bwd --

# 4096 x 4352 x 6144: 272 large tiles, the 16 past the wave take the k-split tail
# (partials summed in order by the reduce kernel, which applies the SwiGLU backward)
# 200 x 128 x 6144: 1 large tile, the whole grid cut along K
@pytest.mark.parametrize("mnk", [(256, 192, 128), (200, 96, 64), (1024, 4864, 896), (4096, 4352, 6144),
                                 (200, 128, 6144)])
def test_swiglu_backward(mnk):
    M, N, Kd = mnk  # rows, intermediate, hidden
    dd = torch.randn(M, Kd, generator=_gen(51)).to(torch.bfloat16)
    wd = torch.randn(Kd, N, generator=_gen(52)).to(torch.bfloat16)
    g = (torch.randn(M, N, generator=_gen(53)) * 3).to(torch.bfloat16)
    u = torch.randn(M, N, generator=_gen(54)).to(torch.bfloat16)
    gu = torch.stack([g.reshape(M, N // 32, 32), u.reshape(M, N // 32, 32)], 2).reshape(M, 2 * N)
    if M * N * Kd > 5e9:  # large case: float32 products on the GPU (their error counted twice)
        ddf, wdf = dd.to(dev()).float(), wd.to(dev()).float()
        dact = (ddf @ wdf).double().cpu()
        abs_prod = (ddf.abs() @ wdf.abs()).double().cpu() * 2
    else:
        dact = dd.double() @ wd.double()
        abs_prod = dd.double().abs() @ wd.double().abs()
    g64, u64 = g.double(), u.double()
    sg = torch.sigmoid(g64)
    dg_ref = dact * u64 * sg * (1 + g64 * (1 - sg))
    du_ref = dact * g64 * sg
    dgu = torch.full((M, 2 * N), 9.0, dtype=torch.bfloat16, device=dev())
    K.gemm_swiglu_bwd(dd.to(dev()), wd.to(dev()), gu.to(dev()), dgu)
    out = dgu.double().cpu().reshape(M, N // 32, 2, 32)
    got_g = out[:, :, 0, :].reshape(M, N)
    got_u = out[:, :, 1, :].reshape(M, N)
    e_act = abs_prod * Kd * 2.0**-23
    tol_g = 1.1 * e_act * u64.abs() + 1e-5 * (dact * u64).abs() + U * dg_ref.abs() + 1e-30
    tol_u = e_act * (g64 * sg).abs() + 1e-5 * du_ref.abs() + U * du_ref.abs() + 1e-30
    assert torch.all((got_g - dg_ref).abs() <= tol_g)
    assert torch.all((got_u - du_ref).abs() <= tol_u)
