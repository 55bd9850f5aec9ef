"""Whole-model scoring on the GPU: the cross-entropy and embedding kernels,
the placed and searched DeltaLoss, the block input gradient, the causal-LM
loss and gradients, and the scoring schedules -- each against the float64
oracle -- and a mixed-precision ``api.quantize`` end to end.

The GPU path rounds logits and GEMM operands to bf16; the stated tolerance for
results computed through bf16 is 1e-2 relative (gradients are compared
normwise, as the block tests compare them). Integer and fp32-elementwise
results (embedding rows, DeltaLoss terms) are exact.
"""

from __future__ import annotations

import json
import sys

import numpy as np
import pytest
import torch

from mround_amd import api
from mround_amd import kernels as K
from mround_amd.core.scale_search import search_scales
from mround_amd.exceptions import KernelError, SchemeError
from mround_amd.pipeline.block import LAYERS, BlockEngine, BlockShape, BlockWeights, placements, unplace
from mround_amd.pipeline.causal_lm import CausalLM
from mround_amd.pipeline.checkpoint import DecoderModel, write_random_checkpoint
from mround_amd.pipeline.runner import DecoderBlock
from mround_amd.pipeline.scoring import score_widths
from mround_amd.planner.allocator import allocate_bits
from mround_amd.planner.sensitivity import mixed_budget_bits, score_layer_options
from mround_amd.schemes import QuantScheme, ScaleInit, Symmetry, TuningConfig
from oracle import block as OB
from oracle import causal_lm as OC
from oracle import sensitivity as OS
from tests.helpers import dev, to_np, weight

pytestmark = pytest.mark.gpu


def _case(*args):
    print("case", *args, flush=True, file=sys.stderr)


# ------------------------------------------------------------ cross-entropy --

@pytest.mark.parametrize("T,V", [(48, 250), (40, 4096), (12, 151936)])
@pytest.mark.parametrize("inplace", [False, True])
def test_cross_entropy(T, V, inplace):
    _case("cross entropy", T, V, inplace)
    g = torch.Generator().manual_seed(V)
    ld = -(-V // 64) * 64
    logits = torch.zeros(T, ld, dtype=torch.bfloat16)
    logits[:, :V] = (torch.randn(T, V, generator=g) * 3).to(torch.bfloat16)
    labels = torch.randint(0, V, (T,), generator=g, dtype=torch.int32)
    labels[3] = -1
    labels[5] = V - 1
    n_valid = int((labels >= 0).sum())
    scale = 1.0 / n_valid
    x = logits[:, :V].double()
    lse = torch.logsumexp(x, 1)
    ref_row = torch.where(labels >= 0, lse - x.gather(1, labels.clamp(min=0).long()[:, None])[:, 0],
                          torch.zeros(()).double())
    onehot = torch.zeros_like(x)
    onehot[labels >= 0] = torch.nn.functional.one_hot(labels[labels >= 0].long(), V).double()
    ref_grad = scale * (torch.softmax(x, 1) - onehot)
    ref_grad[labels < 0] = 0

    ld_ = logits.to(dev())
    lab = labels.to(dev())
    row = torch.empty(T, device=dev())
    loss = torch.empty(1, device=dev())
    dl = ld_ if inplace else torch.zeros_like(ld_)
    K.cross_entropy(ld_, lab, V=V, scale=scale, row_loss=row, loss_out=loss, dlogits=dl)
    got_row = row.double().cpu()
    assert torch.allclose(got_row, ref_row, rtol=1e-6, atol=1e-4), float((got_row - ref_row).abs().max())
    assert float(loss) == pytest.approx(float(ref_row.sum()) * scale, rel=1e-5)
    got = dl.double().cpu()
    err = (got[:, :V] - ref_grad).abs()
    assert bool((err <= ref_grad.abs() * 2.0 ** -8 + 1e-7 * scale).all()), float(err.max())
    assert bool((got[:, V:] == 0).all())  # padding columns untouched
    # a label past the vocabulary is flagged, not read
    bad = labels.clone()
    bad[0] = V
    K.cross_entropy(logits.to(dev()), bad.to(dev()), V=V, scale=scale, row_loss=row)
    assert torch.isnan(row[0]) and not torch.isnan(row[1:]).any()


def test_cross_entropy_rejects_bad_arguments():
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device=dev())
    row = torch.empty(4, device=dev())
    with pytest.raises(KernelError):
        K.cross_entropy(x, torch.zeros(4, dtype=torch.int64, device=dev()), V=64, scale=1.0, row_loss=row)
    with pytest.raises(KernelError):
        K.cross_entropy(x, torch.zeros(4, dtype=torch.int32, device=dev()), V=65, scale=1.0, row_loss=row)


# ---------------------------------------------------------------- embedding --

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H", [136, 100])
def test_embed_rows(dtype, H):
    _case("embed", dtype, H)
    V = 300
    table = torch.randn(V, H, generator=torch.Generator().manual_seed(1)).to(dtype)
    ids = torch.randint(0, V, (77,), generator=torch.Generator().manual_seed(2), dtype=torch.int32)
    ids[4], ids[9] = -1, V
    out = torch.empty(77, H, device=dev())
    K.embed_rows(table.to(dev()), ids.to(dev()), out)
    got = out.cpu()
    ok = (ids >= 0) & (ids < V)
    assert torch.equal(got[ok], table[ids[ok].long()].float())
    assert bool(torch.isnan(got[~ok]).all())


# ---------------------------------------------------------------- DeltaLoss --

@pytest.mark.parametrize("sym", [False, True])
def test_delta_loss_reads_placed_gradients(sym):
    _case("delta mapped", sym)
    rows, cols = 256, 512
    w = weight(rows, cols, seed=3).to(dev())
    g = torch.randn(rows, cols, generator=torch.Generator().manual_seed(4)).to(dev())
    fused = torch.randn(2 * rows, cols, generator=torch.Generator().manual_seed(5)).to(dev())
    view = fused.view(-1, 64, cols)[:, 32:64]
    view.copy_(g.view(-1, 32, cols))
    mode = "sym" if sym else "asym"
    a = torch.zeros(3, dtype=torch.float64, device=dev())
    b = torch.zeros(3, dtype=torch.float64, device=dev())
    K.delta_loss(w, g, group_size=64, bits_list=[2, 3, 4], mode=mode, eps=1e-8, scores_out=a)
    K.delta_loss_mapped(w, fused, group_size=64, bits_list=[2, 3, 4], mode=mode, eps=1e-8, scores_out=b,
                        row_block=32, row_stride=64, row_offset=32)
    assert torch.equal(a, b)


def test_delta_loss_searched_grid():
    _case("delta searched")
    rows, cols, gs = 192, 384, 64
    w = weight(rows, cols, seed=6)
    g = torch.randn(rows, cols, generator=torch.Generator().manual_seed(7))
    grids = []
    want = []
    for bits in (2, 3):
        sch = QuantScheme(bits=bits, group_size=gs, symmetry=Symmetry.SYMMETRIC, scale_init=ScaleInit.SEARCHED)
        grid = search_scales(w.to(dev()), sch).view(rows, cols // gs)
        grids.append(grid)
        w32 = w.float().numpy()
        q = OC.rtn(w32, bits=bits, group_size=gs, mode="searched", init_scale=to_np(grid))
        # the terms in float32, as the scoring pass forms them; the sum in float64
        want.append(float(np.abs(g.numpy() * (q - w32)).astype(np.float64).sum()))
    acc = torch.zeros(2, dtype=torch.float64, device=dev())
    K.delta_loss_mapped(w.to(dev()), g.to(dev()), group_size=gs, bits_list=[2, 3], mode="searched", eps=1e-8,
                        scores_out=acc, grids=grids)
    for i in range(2):
        assert float(acc[i]) == pytest.approx(want[i], rel=1e-9)
    with pytest.raises(KernelError):
        K.delta_loss(w.to(dev()), g.to(dev()), group_size=gs, bits_list=[2], mode="searched", eps=1e-8,
                     scores_out=acc)
    with pytest.raises(KernelError):
        K.delta_loss_mapped(w.to(dev()), g.to(dev()), group_size=gs, bits_list=[2], mode="searched",
                            eps=1e-8, scores_out=acc)


# -------------------------------------------------------- block input grad --

SHAPE = BlockShape(hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, intermediate=256, rope_theta=1e6,
                   attn_bias=True)
SHAPE_D128 = BlockShape(hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, intermediate=512)


def _oshape(s: BlockShape) -> OB.Shape:
    return OB.Shape(hidden=s.hidden, n_heads=s.n_heads, n_kv_heads=s.n_kv_heads, head_dim=s.head_dim,
                    intermediate=s.intermediate, norm_eps=s.norm_eps, rope_theta=s.rope_theta,
                    attn_bias=s.attn_bias)


@pytest.mark.parametrize("shape", [SHAPE, SHAPE_D128], ids=["tiny_qwen", "d128"])
def test_block_input_gradient(shape):
    _case("block dx", shape.hidden)
    B, S = 2, 128
    w = BlockWeights.random(shape, dtype=torch.bfloat16, device="cpu", seed=2, std=0.05)
    gen = torch.Generator().manual_seed(3)
    w.input_norm = 1 + 0.1 * torch.randn(shape.hidden, generator=gen)
    w.post_norm = 1 + 0.1 * torch.randn(shape.hidden, generator=gen)
    x = torch.randn(B * S, shape.hidden, generator=gen)
    r = torch.randn(B * S, shape.hidden, generator=gen)
    xd = x.double().view(B, S, -1).requires_grad_(True)
    out = OB.block_forward(xd, {n: t.double() for n, t in w.linears.items()},
                           {n: t.double() for n, t in w.biases.items()},
                           (w.input_norm.double(), w.post_norm.double()), _oshape(shape))
    (out.reshape(B * S, -1) * r.double()).sum().backward()
    ref = xd.grad.reshape(B * S, -1)

    eng = BlockEngine(shape, batch=B, seq_len=S, device=dev())
    wd = BlockWeights({n: t.to(dev()) for n, t in w.linears.items()}, {n: t.to(dev()) for n, t in w.biases.items()},
                      w.input_norm.to(dev()), w.post_norm.to(dev()))
    eng.set_block(wd)
    eng.load_dense(wd.linears)
    xg = x.to(dev())
    o = torch.empty_like(xg)
    eng.forward(xg, o, save=True)
    eng.grad_out.copy_(r)
    dx = torch.empty_like(xg)
    eng.backward(dx_out=dx)
    got = dx.double().cpu()
    # the residual path carries r itself; measure the error against the block's own part
    err = float((got - ref).norm() / (ref - r.double()).norm())
    print(f"  rel err {err:.2e}", file=sys.stderr)
    assert err < 2e-2


# -------------------------------------------------------------- causal LM --

def _model(kind: str, *, vocab: int, tied: bool, layers: int = 2, seed: int = 0):
    shape = BlockShape(hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, intermediate=256,
                       rope_theta=1e6 if kind == "qwen2" else 1e4, attn_bias=kind == "qwen2")
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    blocks = []
    for i in range(layers):
        w = BlockWeights.random(shape, dtype=bf, device="cpu", seed=seed * 10 + i, std=0.05)
        w.input_norm = 1 + 0.1 * torch.randn(shape.hidden, generator=g)
        w.post_norm = 1 + 0.1 * torch.randn(shape.hidden, generator=g)
        w = BlockWeights({n: t.to(dev()) for n, t in w.linears.items()},
                         {n: t.to(dev()) for n, t in w.biases.items()}, w.input_norm.to(dev()),
                         w.post_norm.to(dev()))
        blocks.append(DecoderBlock(i, f"model.layers.{i}", shape, w))
    embed = (torch.randn(vocab, shape.hidden, generator=g) * 0.5).to(bf).to(dev())
    head = None if tied else (torch.randn(vocab, shape.hidden, generator=g) * 0.5).to(bf).to(dev())
    norm = (1 + 0.1 * torch.randn(shape.hidden, generator=g)).to(dev())
    cfg = {"model_type": kind, "vocab_size": vocab, "num_hidden_layers": layers,
           "tie_word_embeddings": tied}
    return DecoderModel(cfg, bf, embed, blocks, norm, head)


def _oracle_model(m: DecoderModel) -> OC.Model:
    s = m.blocks[0].shape
    blocks = [(b.name, {n: t.double().cpu() for n, t in b.weights.linears.items()},
               {n: t.double().cpu() for n, t in b.weights.biases.items()},
               (b.weights.input_norm.double().cpu(), b.weights.post_norm.double().cpu())) for b in m.blocks]
    return OC.Model(shape=_oshape(s), embed=m.embed.double().cpu(), blocks=blocks, norm=m.norm.double().cpu(),
                    head=None if m.lm_head is None else m.lm_head.double().cpu())


@pytest.mark.parametrize("kind,vocab,tied", [("qwen2", 250, True), ("llama", 320, False)])
def test_causal_lm_loss_and_gradients(kind, vocab, tied):
    _case("causal lm", kind, vocab, tied)
    m = _model(kind, vocab=vocab, tied=tied)
    om = _oracle_model(m)
    tokens = torch.randint(0, vocab, (3, 65), generator=torch.Generator().manual_seed(9))
    lm = CausalLM(m, batch=2, seq_len=65, device=dev())
    lm.set_weights({})
    place = placements(m.blocks[0].shape)
    for batch in (tokens[:2], tokens[2:]):  # a full batch, then a ragged one
        grads = {}

        def grab(b, dw):
            for n in LAYERS:
                rows = m.blocks[b].shape.linear_shape(n)[0]
                grads[f"model.layers.{b}.{n}"] = unplace(dw[place[n].operand], rows, place[n]).double().cpu()

        loss = float(lm.run(batch.to(dev()), grab))
        linears = {f"{name}.{n}": lin[n] for name, lin, *_ in om.blocks for n in LAYERS}
        ref_loss, ref = OC.layer_gradients(om, batch, linears)
        print(f"  loss gpu {loss:.6f} oracle {ref_loss:.6f}", file=sys.stderr)
        assert loss == pytest.approx(ref_loss, rel=1e-2)
        for p, r in ref.items():
            got = grads[p]
            rel = float((got - r).norm() / r.norm())
            flipped = float(r.abs()[torch.sign(got) != torch.sign(r)].sum() / r.abs().sum())
            print(f"  {p}: rel {rel:.2e} flipped {flipped:.2e}", file=sys.stderr)
            assert rel < 5e-2, p
            assert flipped < 1e-2, p


def test_padding_sequences_is_exact():
    """A batch run in a larger engine (extra ignored sequences) gives the same
    loss and gradients as an engine of its own size."""
    _case("causal lm padding")
    m = _model("qwen2", vocab=256, tied=True, layers=1)
    tokens = torch.randint(0, 256, (2, 129), generator=torch.Generator().manual_seed(3)).to(dev())
    out = []
    for batch in (2, 3):
        lm = CausalLM(m, batch=batch, seq_len=129, device=dev())
        lm.set_weights({})
        got = {}
        loss = float(lm.run(tokens, lambda b, dw: got.update({k: v.clone() for k, v in dw.items()})))
        out.append((loss, got))
    assert out[0][0] == pytest.approx(out[1][0], rel=1e-6)
    for k in out[0][1]:
        a, b = out[0][1][k], out[1][1][k]
        assert float((a - b).norm() / a.norm()) < 1e-5, k


# --------------------------------------------------------------- schedules --

@pytest.mark.parametrize("searched", [False, True])
@pytest.mark.parametrize("source", ["own_width", "widest"])
def test_score_widths_match_oracle(searched, source):
    _case("score widths", searched, source)
    m = _model("qwen2", vocab=256, tied=True, layers=2, seed=4)
    om = _oracle_model(m)
    g = torch.Generator().manual_seed(11)
    tokens = torch.randint(0, 256, (3, 129), generator=g)
    batches = [tokens[:2].to(dev()), tokens[2:].to(dev())]
    if searched:
        base = QuantScheme(bits=2, group_size=64, symmetry=Symmetry.SYMMETRIC, scale_init=ScaleInit.SEARCHED)
    else:
        base = QuantScheme(bits=2, group_size=64, symmetry=Symmetry.ASYMMETRIC)
    res = score_widths(m, batches, [2, 4], base, gradient_source=source)
    grids = None
    if searched:
        grids = {}
        for b in (2, 4):
            sch = base.with_bits(b)
            grids[b] = {f"{blk.name}.{n}": to_np(search_scales(blk.weights.linears[n], sch).view(
                blk.weights.linears[n].shape[0], -1)) for blk in m.blocks for n in LAYERS}
    ref = OC.score_widths(om, [t.cpu() for t in batches], [2, 4], group_size=64,
                          mode="searched" if searched else "asym", gradient_source=source, grids=grids)
    assert set(res.scores) == set(ref)
    worst = 0.0
    for p in ref:
        for b in (2, 4):
            rel = abs(res.scores[p][b] - ref[p][b]) / ref[p][b]
            worst = max(worst, rel)
            assert rel < 3e-2, (p, b, res.scores[p][b], ref[p][b])
    print(f"  worst rel {worst:.2e}", file=sys.stderr)
    assert res.shapes["model.layers.0.mlp.down_proj"] == (128, 256)
    _check_plans(res.scores, ref, res.shapes, base, worst)


def _check_plans(gpu, ref, shapes, base, worst):
    """The allocation made from the GPU's scores against the one made from
    the float64 oracle's (mround/planner/allocator.py:98-194) at several
    budgets: the same assignment, or, where scores within ``worst`` of each
    other leave a near-tie, a plan whose DeltaLoss under the oracle's scores
    is within that error of the oracle's optimum."""
    widths = sorted(next(iter(ref.values())))
    for avg in np.linspace(widths[0], widths[-1], 7)[1:-1]:
        budget = mixed_budget_bits(shapes, float(avg), base.group_size)
        a_gpu = allocate_bits(score_layer_options(gpu, shapes, base), budget_bits=budget)
        a_ref = allocate_bits(score_layer_options(ref, shapes, base), budget_bits=budget)
        if a_gpu.by_layer == a_ref.by_layer:
            continue
        under_ref = sum(ref[p][b] for p, b in a_gpu.by_layer.items())
        print(f"  average {avg:.3f}: plans differ; oracle loss of the GPU plan {under_ref:.6g}, "
              f"optimum {a_ref.predicted_loss:.6g}", file=sys.stderr)
        assert under_ref <= a_ref.predicted_loss * (1 + worst) / (1 - worst) + 1e-12


def test_three_width_plan_matches_oracle():
    """Scores at 2, 3 and 4 bits (each width's own gradients) and the plans made
    from them at budgets across the range, against the float64 oracle."""
    _case("plan 2/3/4")
    m = _model("qwen2", vocab=256, tied=True, layers=2, seed=6)
    om = _oracle_model(m)
    tokens = torch.randint(0, 256, (4, 129), generator=torch.Generator().manual_seed(13))
    batches = [tokens[:2].to(dev()), tokens[2:].to(dev())]
    base = QuantScheme(bits=2, group_size=64, symmetry=Symmetry.ASYMMETRIC)
    res = score_widths(m, batches, [2, 3, 4], base, gradient_source="own_width")
    ref = OC.score_widths(om, [t.cpu() for t in batches], [2, 3, 4], group_size=64, mode="asym",
                          gradient_source="own_width")
    worst = max(abs(res.scores[p][b] - ref[p][b]) / ref[p][b] for p in ref for b in (2, 3, 4))
    print(f"  worst rel {worst:.2e}", file=sys.stderr)
    assert worst < 3e-2
    _check_plans(res.scores, ref, res.shapes, base, worst)


def test_schedules_agree_at_the_widest_width():
    _case("schedules agree")
    m = _model("llama", vocab=320, tied=False, layers=2, seed=5)
    tokens = torch.randint(0, 320, (2, 129), generator=torch.Generator().manual_seed(12)).to(dev())
    base = QuantScheme(bits=2, group_size=64, symmetry=Symmetry.ASYMMETRIC)
    own = score_widths(m, [tokens], [2, 4], base, gradient_source="own_width").scores
    wide = score_widths(m, [tokens], [2, 4], base, gradient_source="widest").scores
    for p in own:
        assert own[p][4] == pytest.approx(wide[p][4], rel=1e-9)


# ------------------------------------------------------------ mixed runs --

TINY = dict(model_type="qwen2", hidden_size=128, num_attention_heads=2, num_key_value_heads=1,
            intermediate_size=256, rms_norm_eps=1e-6, rope_theta=1e6, num_hidden_layers=2,
            vocab_size=512, tie_word_embeddings=True)


def test_mixed_quantize_end_to_end(tmp_path):
    _case("api mixed")
    src = write_random_checkpoint(tmp_path / "m", TINY, seed=2, std=0.05)
    tuning = TuningConfig(iters=4, batch_size=2, n_samples=4, seq_len=128)
    kw = dict(bits=4, symmetry=Symmetry.ASYMMETRIC, average_bits=3.0, candidate_bits=(2, 4),
              scoring_samples=4, scoring_seq_len=129, seed=3)
    res = api.quantize(src, output_dir=tmp_path / "q", tuning=tuning, **kw)
    mixed = res.mixed
    assert mixed["source"] == "scored" and mixed["gradient_source"] == "widest"
    assert mixed["scoring_batch_size"] == 4  # 2048 tokens per batch hold all four sequences
    assert mixed["allocated_cost_bits"] <= mixed["budget_bits"]
    assert mixed["remainder_bits"] == 3
    assign = mixed["assignments"]
    assert set(assign.values()) <= {2, 4} and len(assign) == 14
    cfg = json.loads((tmp_path / "q" / "config.json").read_text())
    q = cfg["quantization"]
    for path, bits in assign.items():
        assert q.get(path, q)["bits"] == bits
    assert q.get("model.embed_tokens", q)["bits"] == 3
    record = json.loads((tmp_path / "q" / "mround_run.json").read_text())
    assert record["mixed"]["assignments"] == assign
    plan = api.plan_mixed_precision(src, 3.0, (2, 4), bits=4, symmetry=Symmetry.ASYMMETRIC,
                                    scoring_samples=4, scoring_seq_len=129, seed=3)
    assert plan["assignments"] == assign
    # the same plan given back is costed identically and tunes the same widths
    res2 = api.quantize(src, output_dir=tmp_path / "q2", tuning=tuning, plan=assign,
                        **{k: v for k, v in kw.items() if not k.startswith("scoring")})
    assert res2.mixed["source"] == "given"
    assert res2.mixed["allocated_cost_bits"] == mixed["allocated_cost_bits"]
    with pytest.raises(SchemeError, match="exactly the block layers"):
        api.quantize(src, output_dir=tmp_path / "q3", tuning=tuning,
                     plan={k: v for k, v in list(assign.items())[1:]},
                     **{k: v for k, v in kw.items() if not k.startswith("scoring")})
