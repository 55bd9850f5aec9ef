"""The benchmark configurations' kernels and block tune at their full sizes.

* The kernel microbench matrix: one bf16 18944 x 3584 weight N(0, 0.02) with
  0.1 % of entries x10 (seed 0), v U(-0.5, 0.5) (seed 2), alpha = beta = 1,
  dL/dW' N(0, 1) fp32 (seed 3), asymmetric, at every bits x group size point
  of the sweep (2/3/4/8 x 32/64/128). On sampled rows, against the float32
  oracle: the forward (W', codes, scale, zero point) and the packed words bit
  for bit, and the fused quantize + pack of the export identical to them; the fused sign-SGD step (v bit for bit, alpha and beta wherever the
  gradient's sign is clear of its summation-order error) and the next W' it
  writes, bit-identical to the oracle forward of the parameters it wrote. The
  step without the W' write leaves the same parameters over the whole matrix.
* The outlier threshold at the Qwen2.5-7B batch (8 x 2048 x 3584 =
  58,720,256 residuals, k = 58,720): the exact k-th largest |r| against
  NumPy's partition, and the loss against a float64 sum.
* The Qwen2.5-7B-shaped block (hidden 3584, 28 / 4 heads x 128, SwiGLU
  18944, q/k/v biases, bf16 N(0, 0.02) weights), 128 x 2048 uniform token
  ids through a random embedding, 2-bit asymmetric gs64, 200 steps at batch
  8 with the outlier rule: the whole block tune twice (identical codes and
  losses), the loss falls and the revert rule holds, codes in range, and the
  committed codes, scales, zero points and reconstruction bit-exact with the
  oracle's forward of the final parameters on sampled rows; and the first
  step (round-to-nearest W') on a one-sequence slice of 512 tokens against
  the float64 block: the loss within the 1e-2 bar, every layer's dL/dW'
  within 5 % normwise with under 1 % of its mass changing sign (the update
  takes signs).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from mround_amd import kernels as K
from mround_amd.core import quantizer as QZ
from mround_amd.formats import mlx_export as MX
from mround_amd.formats import packing as PK
from mround_amd.pipeline.block import LAYERS, BlockEngine, BlockShape, BlockWeights, placements, unplace
from mround_amd.pipeline.runner import DecoderBlock, QuantizationRunner
from mround_amd.schemes import QuantScheme, Symmetry, TuningConfig
from oracle import block as OB
from oracle import packing as OP
from oracle import quantize as OQ
from tests.helpers import dev, to_np, weight
from tests.test_gpu_quant import _grad_tolerance

pytestmark = pytest.mark.gpu

ROWS, COLS = 18944, 3584
SEL = np.r_[0:32, 9472:9504, ROWS - 32:ROWS]  # sampled rows: top, middle, bottom


def _note(*case):
    print("case", *case, flush=True, file=sys.stderr)


@pytest.fixture(scope="module")
def micro():
    w = weight(ROWS, COLS, seed=0)
    v = torch.rand(ROWS, COLS, generator=torch.Generator().manual_seed(2)) - 0.5
    g = torch.randn(ROWS, COLS, generator=torch.Generator().manual_seed(3))
    return {"w": w, "v": v, "g": g, "wd": w.to(dev()), "vd": v.to(dev()), "gd": g.to(dev()),
            "w_np": to_np(w)[SEL], "v_np": v.numpy()[SEL], "g_np": g.numpy()[SEL]}


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_microbench_matrix(micro, bits, gs):
    _note("microbench", bits, gs)
    ng = COLS // gs
    wd, gd = micro["wd"], micro["gd"]
    v = micro["vd"].clone()
    a = torch.ones(ROWS, ng, device=dev())
    b = torch.ones(ROWS, ng, device=dev())
    w_np, v_np, g_np = micro["w_np"], micro["v_np"], micro["g_np"]
    ones = np.ones((len(SEL), ng), dtype=np.float32)

    # forward: W', codes, scale, zero point
    wq = torch.empty(ROWS, COLS, dtype=torch.bfloat16, device=dev())
    codes = torch.empty(ROWS, ng, gs, dtype=torch.uint8, device=dev())
    scale = torch.empty(ROWS, ng, device=dev())
    zp = torch.empty(ROWS, ng, device=dev())
    K.fq_forward(wd, v, a, b, bits=bits, group_size=gs, mode="asym", eps=1e-8, wq_out=wq, codes_out=codes,
                 scale_out=scale, zp_out=zp)
    ref_q, ref_c, ref_s, ref_z = OQ.fake_quantize(w_np, v_np, ones, ones, bits=bits, group_size=gs,
                                                  mode="asym", dtype=np.float32)
    assert np.array_equal(to_np(wq)[SEL], OQ.round_to_bf16(ref_q)), "W' differs"
    assert np.array_equal(to_np(codes)[SEL].astype(np.int64).reshape(len(SEL), -1),
                          ref_c.astype(np.int64).reshape(len(SEL), -1)), "codes differ"
    assert np.array_equal(to_np(scale)[SEL], ref_s.reshape(len(SEL), ng)), "scales differ"
    assert np.array_equal(to_np(zp)[SEL], ref_z.reshape(len(SEL), ng)), "zero points differ"
    assert int(codes.max()) <= 2**bits - 1

    # packing of the whole matrix; sampled rows against the oracle's words
    packed = PK.pack_codes(codes.view(ROWS, COLS), bits)
    want = OP.pack_codes(ref_c.reshape(len(SEL), COLS).astype(np.int64), bits)
    assert np.array_equal(packed.view(torch.int32).cpu().numpy().view(np.uint32)[SEL], want), "packed words"
    # the fused quantize + pack of the export: the same words, and the affine metadata, over the whole matrix
    scheme = QuantScheme(bits=bits, group_size=gs, symmetry=Symmetry.ASYMMETRIC)
    params = {"v": v.view(ROWS, ng, gs), "alpha": a.view(ROWS, ng, 1), "beta": b.view(ROWS, ng, 1)}
    words, scl, bia = QZ.quantize_pack(wd, params, scheme, dtype=torch.bfloat16)
    assert torch.equal(words.view(torch.int32), packed.view(torch.int32)), "fused words"
    ws_, wb_ = MX.to_affine(scale, zp, scheme, dtype=torch.bfloat16)
    assert torch.equal(scl, ws_.reshape(ROWS, ng)) and torch.equal(bia, wb_.reshape(ROWS, ng)), "fused metadata"

    # the fused step that also writes the next W' (identity placement)
    lr = 0.005
    wq2 = torch.empty(ROWS, COLS, dtype=torch.bfloat16, device=dev())
    K.fq_step_requant_mapped(wd, v, a, b, gd, bits=bits, group_size=gs, mode="asym", eps=1e-8, lr=lr,
                             coef_lo=0.1, coef_hi=1.0, v_bound=0.5, row_block=0, row_stride=0, row_offset=0,
                             wq_out=wq2)
    gv, ga, gb = OQ.quantize_grad(w_np, v_np, ones, ones, g_np, bits=bits, group_size=gs, mode="asym",
                                  dtype=np.float32)
    ref_v = np.clip(v_np - np.float32(lr) * np.sign(gv).reshape(v_np.shape), -0.5, 0.5)
    assert np.array_equal(to_np(v)[SEL], ref_v), "updated v differs"
    ss, sd = _grad_tolerance(w_np, v_np, ones, ones, g_np, bits, gs, "asym", None)
    tol = ((gs / 64 + 16) * np.finfo(np.float32).eps * (ss + sd)).reshape(len(SEL), ng)
    for name, got, grad in (("alpha", a, ga), ("beta", b, gb)):
        grad = grad.reshape(len(SEL), ng)
        ref_new = np.clip(np.float32(1.0) - np.float32(lr) * np.sign(grad), 0.1, 1.0)
        clear = np.abs(grad) > tol
        assert clear.mean() > 0.8  # (89-97 % at 8 bits, where the bound is widest)
        assert np.array_equal(to_np(got)[SEL][clear], ref_new[clear]), f"updated {name} differs"
    # the W' written is the oracle forward of the parameters written
    nq, _, _, _ = OQ.fake_quantize(w_np, to_np(v)[SEL], to_np(a)[SEL], to_np(b)[SEL], bits=bits,
                                   group_size=gs, mode="asym", dtype=np.float32)
    assert np.array_equal(to_np(wq2)[SEL], OQ.round_to_bf16(nq)), "requantized W' differs"

    # the plain fused step (no W' write) leaves the same parameters everywhere
    v3 = micro["vd"].clone()
    a3 = torch.ones(ROWS, ng, device=dev())
    b3 = torch.ones(ROWS, ng, device=dev())
    K.fq_backward_signsgd(wd, v3, a3, b3, gd, bits=bits, group_size=gs, mode="asym", eps=1e-8, update=True,
                          lr=lr, coef_lo=0.1, coef_hi=1.0, v_bound=0.5)
    assert torch.equal(v3, v) and torch.equal(a3, a) and torch.equal(b3, b)


def test_outlier_threshold_at_the_7b_batch():
    n = 8 * 2048 * 3584
    k = max(1, int(n * 0.001))
    _note("outlier threshold", n, k)
    g = torch.Generator(device=dev()).manual_seed(8)
    target = torch.randn(n, generator=g, device=dev())
    pred = target + torch.randn(n, generator=g, device=dev()) * 0.05
    pred[::1000] += 3.0  # a heavy tail of 58,721 large residuals
    loss = torch.empty(1, device=dev())
    thr = torch.empty(1, device=dev())
    grad = torch.empty(n, device=dev())
    K.loss_outlier(pred, target, k=k, denom=n, loss_out=loss, threshold_out=thr, grad_out=grad)
    r = (pred - target).abs().cpu().numpy()
    kth = np.partition(r, n - k)[n - k]
    assert float(thr) == float(kth)
    kept = r < kth
    want = float(np.sum(r[kept].astype(np.float64) ** 2) / n)
    assert float(loss) == pytest.approx(want, rel=1e-6)
    gsel = grad[:1 << 20].cpu().numpy()
    rs = (pred - target)[:1 << 20].cpu().numpy()
    assert np.array_equal(gsel, np.where(np.abs(rs) < kth, rs * np.float32(2.0 / n), 0).astype(np.float32))


# ------------------------------------------------------- the 7B block tune --

SHAPE_7B = BlockShape(hidden=3584, n_heads=28, n_kv_heads=4, head_dim=128, intermediate=18944,
                      norm_eps=1e-6, rope_theta=1e6, attn_bias=True)
VOCAB = 152064


def layer_rows(n_rows: int) -> np.ndarray:
    """Sampled rows of a layer with ``n_rows`` rows: its first and last 16
    (checked on the host, before any device indexing)."""
    sel = np.unique(np.r_[0:16, n_rows - 16:n_rows])
    assert 0 <= sel.min() and sel.max() < n_rows
    return sel


def _block_7b():
    w = BlockWeights.random(SHAPE_7B, dtype=torch.bfloat16, device=dev(), seed=0)
    tokens = torch.randint(0, VOCAB, (128, 2048), generator=torch.Generator(device=dev()).manual_seed(6),
                           device=dev())
    embed = (torch.randn(VOCAB, SHAPE_7B.hidden, generator=torch.Generator(device=dev()).manual_seed(7),
                         device=dev()) * 0.02).to(torch.bfloat16)
    entrance = [embed[tokens[i:i + 8].reshape(-1)].float() for i in range(0, 128, 8)]
    return w, entrance


def _tune_7b(w, entrance):
    scheme = QuantScheme(bits=2, group_size=64, symmetry=Symmetry.ASYMMETRIC)
    runner = QuantizationRunner(scheme, TuningConfig(iters=200, batch_size=8, n_samples=128, seq_len=2048))
    block = DecoderBlock(0, "model.layers.0", SHAPE_7B,
                         BlockWeights(dict(w.linears), w.biases, w.input_norm, w.post_norm))
    final = {}
    commit = runner._commit

    def spy(blk, layer):
        sel = layer_rows(layer.v.shape[0])
        final[layer.name] = tuple(t[sel].cpu().numpy().copy() for t in (layer.v, layer.alpha, layer.beta))
        return commit(blk, layer)

    runner._commit = spy
    summary, layers = runner.run([block], [x.clone() for x in entrance])
    torch.cuda.synchronize()
    return summary.blocks[0], layers, final, block


def test_7b_block_tune_at_full_size():
    _note("7b block tune")
    w, entrance = _block_7b()
    res, layers, final, block = _tune_7b(w, entrance)
    print(f"  loss {res.initial_loss:.6g} -> {res.final_loss:.6g}, reverted {res.reverted}, "
          f"{res.seconds:.2f} s", file=sys.stderr)
    # the revert rule, and learning
    assert res.reverted == (res.final_loss >= res.initial_loss)
    assert not res.reverted and res.final_loss < 0.8 * res.initial_loss
    losses = np.asarray(res.step_losses)
    assert np.all(np.isfinite(losses)) and losses[-16:].mean() < losses[:16].mean()
    for n in LAYERS:
        q = layers[f"model.layers.0.{n}"]
        rows, cols = w.linears[n].shape
        assert q.codes.shape == (rows, cols // 64, 64) and int(q.codes.max()) <= 3
        # committed codes, scales, zero points and reconstruction: the oracle's
        # forward of the final parameters, bit for bit
        v, a, b = final[n]
        sel = layer_rows(rows)
        wn = w.linears[n][sel].float().cpu().numpy()
        ref_q, ref_c, ref_s, ref_z = OQ.fake_quantize(wn, v, a, b, bits=2, group_size=64, mode="asym",
                                                      dtype=np.float32)
        assert np.array_equal(q.codes[sel].cpu().numpy().astype(np.float32),
                              ref_c.reshape(len(sel), -1, 64)), n
        assert np.array_equal(q.scale[sel].cpu().numpy().reshape(-1), ref_s.reshape(-1)), n
        assert np.array_equal(q.zero_point[sel].cpu().numpy().reshape(-1), ref_z.reshape(-1)), n
        assert np.array_equal(block.weights.linears[n][sel].float().cpu().numpy(),
                              OQ.round_to_bf16(ref_q)), n
    # a second run commits the same codes and losses
    res2, layers2, _, _ = _tune_7b(w, entrance)
    assert res2.step_losses == res.step_losses and res2.final_loss == res.final_loss
    for path, q in layers.items():
        assert torch.equal(q.codes, layers2[path].codes), path


def _oshape(s: BlockShape) -> OB.Shape:
    return OB.Shape(hidden=s.hidden, n_heads=s.n_heads, n_kv_heads=s.n_kv_heads, head_dim=s.head_dim,
                    intermediate=s.intermediate, norm_eps=s.norm_eps, rope_theta=s.rope_theta,
                    attn_bias=s.attn_bias)


def test_7b_first_step_on_a_slice_against_float64():
    """The first tuning step (W' = 2-bit round to nearest, the outlier rule on)
    over the first 512 tokens of one calibration sequence: the loss and every
    layer's dL/dW' against float64 autograd through the same W'."""
    _note("7b first step slice")
    torch.set_num_threads(16)
    S = 512
    w, entrance = _block_7b()
    x = entrance[0][:S].clone()
    del entrance
    scheme = QuantScheme(bits=2, group_size=64, symmetry=Symmetry.ASYMMETRIC)
    wq = {n: QZ.fake_quantize(w.linears[n], None, scheme, out_dtype=torch.bfloat16) for n in LAYERS}
    eng = BlockEngine(SHAPE_7B, batch=1, seq_len=S, device=dev())
    eng.set_block(w)
    eng.load_dense(wq)
    out = torch.empty_like(x)
    eng.forward(x, out, save=True)
    t64 = _oracle_target(w, x, S)
    got_loss = float(eng.loss(out, t64.float().to(dev()), suppress=True, with_grad=True))
    eng.backward()
    # float64 over the same W'
    lin = {n: wq[n].double().cpu().requires_grad_(True) for n in LAYERS}
    biases = {n: t.double().cpu() for n, t in w.biases.items()}
    norms = (w.input_norm.double().cpu(), w.post_norm.double().cpu())
    pred = OB.block_forward(x.double().cpu().view(1, S, -1), lin, biases, norms, _oshape(SHAPE_7B))
    loss, dpred = OB.batch_loss(pred.detach().reshape(S, -1), t64.reshape(S, -1), True)
    pred.backward(dpred.view_as(pred))
    print(f"  loss gpu {got_loss:.6e} float64 {float(loss):.6e}", file=sys.stderr)
    assert abs(got_loss - float(loss)) <= 1e-2 * float(loss)
    place = placements(SHAPE_7B)
    for n in LAYERS:
        ref = lin[n].grad
        got = unplace(eng.dw[place[n].operand], ref.shape[0], place[n]).double().cpu()
        rel = float((got - ref).norm() / ref.norm())
        flipped = float(ref.abs()[torch.sign(got) != torch.sign(ref)].sum() / ref.abs().sum())
        print(f"  {n}: rel err {rel:.2e}, flipped mass {flipped:.2e}", file=sys.stderr)
        assert rel < 5e-2, n
        assert flipped < 1e-2, n


def _oracle_target(w, x, S):
    lin = {n: t.double().cpu() for n, t in w.linears.items()}
    biases = {n: t.double().cpu() for n, t in w.biases.items()}
    norms = (w.input_norm.double().cpu(), w.post_norm.double().cpu())
    with torch.no_grad():
        return OB.block_forward(x.double().cpu().view(1, S, -1), lin, biases, norms,
                                _oshape(SHAPE_7B)).reshape(S, -1)
