"""Block-by-block SignRound tuning on one GPU.

The host side of ``QuantizationRunner`` (mround/pipeline/runner.py:427-953):
the targets pass over the original weights, the tuning loop (score every
batch, ``iters`` sign-SGD steps on cycled batches, score again, revert to
round to nearest when the score did not improve), the commit of codes and
reconstructions, and the advance of the quantized stream. Every array lives
on the device; the loop issues kernels on the current stream and reads back
one scalar per scored batch set, none per step.
"""

from __future__ import annotations

import dataclasses
import time
from collections.abc import Callable, Mapping, Sequence

import torch

from mround_amd import kernels as K
from mround_amd.core.quantizer import fake_quantize, mode_of, quantize_codes
from mround_amd.core.scale_search import search_scales
from mround_amd.core.signsgd import LinearDecay
from mround_amd.exceptions import ArchitectureError, CalibrationError
from mround_amd.formats.mlx_export import QuantizedLayer
from mround_amd.pipeline.block import (LAYERS, BlockEngine, BlockShape, BlockWeights, aligned_length, placements,
                                       unplace)
from mround_amd.pipeline.block import place as place_rows
from mround_amd.schemes import DEFAULT_EPS_FP32, QuantScheme, ScaleInit, TuningConfig

V_BOUND = 0.5
# Steps replay recorded graphs when a batch is at most this many
# (token x hidden) elements and each batch's graph would replay at least
# GRAPH_MIN_REPLAYS times (see QuantizationRunner._use_graphs).
GRAPH_MAX_ELEMENTS = 4096 * 1024
GRAPH_MIN_REPLAYS = 20


def piece_bounds(size: int, pieces: int) -> list[tuple[int, int]]:
    """``size`` sequences in at most ``pieces`` contiguous runs, none empty,
    the first ones a sequence longer where they cannot be equal
    (mround/pipeline/blocks.py:609-624)."""
    count = max(1, min(pieces, size))
    base, extra = divmod(size, count)
    bounds, start = [], 0
    for i in range(count):
        stop = start + base + (1 if i < extra else 0)
        bounds.append((start, stop))
        start = stop
    return bounds


@dataclasses.dataclass
class DecoderBlock:
    """One block of a model: its position, dotted name, geometry and weights."""

    index: int
    name: str
    shape: BlockShape
    weights: BlockWeights


@dataclasses.dataclass(frozen=True)
class BlockResult:
    """What tuning one block achieved (mround/pipeline/runner.py:188-260)."""

    index: int
    name: str
    initial_loss: float
    final_loss: float
    iterations: int
    seconds: float
    tuned: tuple[str, ...]
    skipped: tuple[tuple[str, str], ...] = ()
    reverted: bool = False
    generalization_gap: float | None = None
    search_seconds: float = 0.0
    stage_seconds: Mapping[str, float] = dataclasses.field(default_factory=dict)
    step_losses: tuple[float, ...] = ()

    @property
    def improvement(self) -> float:
        if self.initial_loss <= 0:
            return 0.0
        return 1.0 - self.final_loss / self.initial_loss


@dataclasses.dataclass(frozen=True)
class RunSummary:
    blocks: list[BlockResult]
    total_seconds: float
    peak_memory_bytes: int
    scheme_by_layer: Mapping[str, QuantScheme]

    @property
    def mean_improvement(self) -> float:
        if not self.blocks:
            return 0.0
        return sum(b.improvement for b in self.blocks) / len(self.blocks)


def block_recipe(tuning: TuningConfig, base_bits: int, widths: Mapping[str, int], *,
                 per_layer: bool) -> tuple[bool, dict[str, float]]:
    """Outlier rule and per-layer initial rate (mround/pipeline/runner.py:389-425)."""
    if not per_layer:
        rate = tuning.resolved_lr(base_bits)
        return tuning.resolved_suppress_outliers(base_bits), dict.fromkeys(widths, rate)
    narrowest = min(widths.values(), default=base_bits)
    return tuning.resolved_suppress_outliers(narrowest), {
        name: tuning.resolved_lr(bits) for name, bits in widths.items()
    }


class _Layer:
    """A linear being tuned: the original weight (model dtype, never updated),
    its scheme, its rows' place in the fused operand, and (v, alpha, beta)."""

    def __init__(self, name: str, weight: torch.Tensor, scheme: QuantScheme, placement) -> None:
        self.name = name
        self.weight = weight.contiguous()
        self.scheme = scheme
        self.mode = mode_of(scheme)
        self.placement = placement
        rows, cols = weight.shape
        ng = 1 if scheme.group_size == -1 else cols // scheme.group_size
        dev = weight.device
        self.v = torch.zeros(rows, cols, dtype=torch.float32, device=dev)
        self.alpha = torch.ones(rows, ng, dtype=torch.float32, device=dev)
        self.beta = torch.ones(rows, ng, dtype=torch.float32, device=dev)
        self.init_scale: torch.Tensor | None = None  # (rows, ng) fp32 for a searched scheme

    def params(self) -> dict[str, torch.Tensor]:
        rows, cols = self.weight.shape
        gs = cols if self.scheme.group_size == -1 else self.scheme.group_size
        return {"v": self.v.view(rows, -1, gs), "alpha": self.alpha.unsqueeze(-1),
                "beta": self.beta.unsqueeze(-1)}

    def snapshot(self):
        return self.v.clone(), self.alpha.clone(), self.beta.clone()

    def restore(self, saved) -> None:
        for dst, src in zip((self.v, self.alpha, self.beta), saved):
            dst.copy_(src)


class QuantizationRunner:
    """Walks a model block by block, quantizing each in turn."""

    def __init__(self, scheme: QuantScheme, tuning: TuningConfig, *,
                 progress: Callable[[BlockResult], None] | None = None,
                 eps: float = DEFAULT_EPS_FP32, quantized_inputs: bool = True,
                 holdout_batches: int = 0, per_layer_recipe: bool = False,
                 graphs: bool | None = None, fused_advance: bool = True,
                 split_precision: bool = False) -> None:
        if holdout_batches < 0:
            msg = f"holdout_batches must be zero or more, got {holdout_batches}"
            raise CalibrationError(msg)
        self.scheme = scheme
        self.tuning = tuning
        self.progress = progress
        self.eps = eps
        self.quantized_inputs = quantized_inputs
        self.holdout_batches = holdout_batches
        self.per_layer_recipe = per_layer_recipe
        self.graphs = graphs  # None: decided per block (see _use_graphs)
        # With a quantized stream and no held-out batches, the final score is
        # taken from the advance pass (see run); False scores separately.
        self.fused_advance = fused_advance
        # The forward's products in split precision (BlockEngine's split): the
        # block objective to about 16 significant bits in place of bf16's 8.
        self.split = bool(split_precision)
        self._engines: dict = {}
        # rows per sequence in the streams: seq_len rounded up to the attention
        # tile, the rows past seq_len padding (see BlockEngine)
        self.rows = aligned_length(tuning.seq_len)

    def _scheme_for(self, path: str, overrides: Mapping[str, QuantScheme] | None) -> QuantScheme:
        if overrides is None:
            return self.scheme
        return overrides.get(path, self.scheme)

    def engine(self, shape: BlockShape, tokens: int, device) -> BlockEngine:
        """The block engine for this geometry, built once per run: for a batch
        of ``tokens`` tokens, or for its largest piece when steps run in
        pieces (``TuningConfig.micro_batches``)."""
        seq = self.rows
        if tokens % seq:
            raise CalibrationError(f"a batch of {tokens} rows is not whole sequences of {seq}")
        n_seq = tokens // seq
        capacity = max(hi - lo for lo, hi in piece_bounds(n_seq, self.tuning.micro_batches))
        key = (shape, capacity, str(device))
        eng = self._engines.get(key)
        if eng is None:
            eng = BlockEngine(shape, batch=capacity, seq_len=seq, device=device, real_len=self.tuning.seq_len,
                              split=self.split)
            self._engines = {key: eng}
        return eng

    def _pieces(self, x: torch.Tensor) -> list[tuple[int, int]]:
        """Row ranges of a batch's pieces."""
        seq = self.rows
        return [(lo * seq, hi * seq) for lo, hi in piece_bounds(x.shape[0] // seq, self.tuning.micro_batches)]

    def _forward(self, eng: BlockEngine, x: torch.Tensor, out: torch.Tensor) -> None:
        """``out = block(x)`` for a whole batch (no activations kept), a piece at
        a time when the engine holds pieces; ``out`` may be ``x``."""
        seq = self.rows
        for lo, hi in self._pieces(x):
            eng.set_sequences((hi - lo) // seq)
            eng.forward(x[lo:hi], out[lo:hi], save=False)

    # ------------------------------------------------------------------ run --
    def run(self, blocks: Sequence[DecoderBlock], entrance: Sequence[torch.Tensor], *,
            scheme_by_layer: Mapping[str, QuantScheme] | None = None):
        """Quantize every block in place (mround/pipeline/runner.py:493-625).

        ``entrance`` holds the first block's input hidden states, one float32
        ``[batch * rows, hidden]`` device tensor per calibration batch, where
        ``rows`` (``self.rows``) is ``seq_len`` rounded up to a multiple of 128
        and each sequence's rows past ``seq_len`` are padding; the list is
        consumed (its tensors are overwritten by the streams).
        """
        started = time.perf_counter()
        if not entrance:
            raise CalibrationError("no calibration batches")
        reference_stream = [x.float().contiguous() for x in entrance]
        quantized_stream = [x.clone() for x in reference_stream] if self.quantized_inputs else None
        # The final score and the advance run the same forward (the tuned W'
        # equals the committed reconstruction bit for bit) over the same
        # stream, so with no held-out batches one pass does both: the advance
        # writes into a spare stream and scores each batch against its target;
        # a revert re-commits round to nearest and advances again from the
        # untouched inputs. Identical losses, codes and streams, one pass over
        # the calibration set fewer per block. (A float16 model's committed
        # reconstruction is rounded through float16, so its W' is not the
        # tuned one: there the final score is taken separately. So it is in
        # split precision, whose scores read W' to about 16 bits while the
        # committed reconstruction is bf16.)
        half = any(w.dtype == torch.float16 for b in blocks for w in b.weights.linears.values())
        fused = (quantized_stream is not None and self.fused_advance and self.holdout_batches == 0
                 and not half and not self.split)
        spare = [torch.empty_like(x) for x in quantized_stream] if fused else None
        # Without a quantized stream the targets are a second stream; the two
        # trade places after each block, so two streams are held in all.
        free_targets = None
        results, exported, schemes = [], {}, {}
        for block in blocks:
            t0 = time.perf_counter()
            eng = self.engine(block.shape, reference_stream[0].shape[0], reference_stream[0].device)
            eng.set_block(block.weights)
            # Targets: the original block over the reference stream, written over
            # it when the quantized stream carries the inputs (two streams resident).
            eng.load_dense(block.weights.linears)
            if quantized_stream is not None:
                targets = reference_stream
                for x in targets:
                    self._forward(eng, x, x)
            else:
                targets = free_targets or [torch.empty_like(x) for x in reference_stream]
                for x, out in zip(reference_stream, targets):
                    self._forward(eng, x, out)
            torch.cuda.synchronize(eng.device)
            targets_seconds = time.perf_counter() - t0
            inputs = quantized_stream if quantized_stream is not None else reference_stream
            pending = None
            if fused:
                result, layers, pending = self._quantize_block(
                    block, inputs, targets, scheme_by_layer=scheme_by_layer, path_prefix=block.name,
                    defer_final=True)
            else:
                result, layers = self.quantize_block(block, inputs, targets, scheme_by_layer=scheme_by_layer,
                                                     path_prefix=block.name)
            t1 = time.perf_counter()
            if pending is not None:
                final = self._advance(eng, block, quantized_stream, spare, targets, pending["suppress"])
                reverted = final >= pending["initial"]
                if reverted:
                    for name, layer in pending["layers"].items():
                        layer.restore(pending["start"][name])
                        # the tuned commit's codes and reconstruction go first, so that
                        # the round-to-nearest commit reuses their memory
                        layers.pop(f"{block.name}.{name}", None)
                        block.weights.linears[name] = layer.weight
                        layers[f"{block.name}.{name}"] = self._commit(block, layer)
                    self._advance(eng, block, quantized_stream, spare, None, pending["suppress"])
                quantized_stream, spare = spare, quantized_stream
                result = dataclasses.replace(
                    result, final_loss=pending["initial"] if reverted else final, reverted=reverted,
                    seconds=result.seconds + (time.perf_counter() - t1))
            elif quantized_stream is not None:
                eng.load_dense(block.weights.linears)
                for x in quantized_stream:
                    self._forward(eng, x, x)
            exported.update(layers)
            for path in layers:
                schemes[path] = self._scheme_for(path, scheme_by_layer)
            torch.cuda.synchronize(eng.device)
            stages = dict(result.stage_seconds)
            stages["targets"] = targets_seconds
            stages["advance"] = time.perf_counter() - t1
            result = dataclasses.replace(result, stage_seconds=stages)
            if quantized_stream is None:
                free_targets = reference_stream  # this block's inputs, free once its outputs exist
            reference_stream = targets
            results.append(result)
            if self.progress is not None:
                self.progress(result)
        peak = torch.cuda.max_memory_allocated() if torch.cuda.is_available() else 0
        return RunSummary(results, time.perf_counter() - started, peak, schemes), exported

    # -------------------------------------------------------- quantize_block --
    def quantize_block(self, block: DecoderBlock, inputs: Sequence[torch.Tensor],
                       targets: Sequence[torch.Tensor], *,
                       scheme_by_layer: Mapping[str, QuantScheme] | None = None,
                       path_prefix: str = ""):
        """Tune and commit one block (mround/pipeline/runner.py:627-710). The
        block's linears are replaced by their reconstructions in the model dtype."""
        result, exported, _ = self._quantize_block(block, inputs, targets, scheme_by_layer=scheme_by_layer,
                                                   path_prefix=path_prefix)
        return result, exported

    def _quantize_block(self, block: DecoderBlock, inputs, targets, *, scheme_by_layer=None,
                        path_prefix: str = "", defer_final: bool = False):
        """``quantize_block``; with ``defer_final`` the final score and the
        revert decision are left to the caller (returned as the third item:
        the initial score, the loss form, the layers and their starting
        parameters), and the result's final loss is provisional."""
        started = time.perf_counter()
        place = placements(block.shape)
        layers: dict[str, _Layer] = {}
        skipped = []
        for name in LAYERS:
            path = f"{path_prefix}.{name}" if path_prefix else name
            scheme = self._scheme_for(path, scheme_by_layer)
            w = block.weights.linears[name]
            if scheme.group_size > 0 and w.shape[-1] % scheme.group_size:
                skipped.append((name, f"last dimension {w.shape[-1]} is not a multiple of "
                                      f"{scheme.group_size}"))
                continue
            layers[name] = _Layer(name, w, scheme, place[name])
        if not layers:
            reasons = "; ".join(f"{n}: {why}" for n, why in skipped)
            raise ArchitectureError(f"nothing in {block.name!r} can be quantized at this group size, so the "
                                    f"block would be left at full precision without saying so. {reasons}")

        eng = self.engine(block.shape, inputs[0].shape[0], inputs[0].device)
        eng.set_block(block.weights)
        t_search = time.perf_counter()
        searched = self._search_scales(eng, block, layers, inputs)
        search_seconds = time.perf_counter() - t_search if searched else 0.0
        # Layers left dense keep their weight (rounded to bf16) in the fused
        # operands; the tuned layers' rows are rewritten every step.
        for name, _ in skipped:
            p = place[name]
            if eng.split:
                place_rows(eng.w32[p.operand], block.weights.linears[name].float(), p)
            else:
                place_rows(eng.wq[p.operand], block.weights.linears[name].to(torch.bfloat16), p)
        outcome = self._tune(eng, layers, inputs, targets, defer_final=defer_final)
        t_commit = time.perf_counter()
        exported = {}
        for name, layer in layers.items():
            path = f"{path_prefix}.{name}" if path_prefix else name
            exported[path] = self._commit(block, layer)
        torch.cuda.synchronize(eng.device)
        stages = dict(outcome["stages"])
        stages["commit"] = time.perf_counter() - t_commit
        result = BlockResult(
            index=block.index, name=block.name, initial_loss=outcome["initial"],
            final_loss=outcome["final"], iterations=self.tuning.iters,
            seconds=time.perf_counter() - started, tuned=tuple(sorted(layers)),
            skipped=tuple(skipped), reverted=outcome["reverted"], generalization_gap=outcome["gap"],
            search_seconds=search_seconds, stage_seconds=stages, step_losses=tuple(outcome["losses"]))
        pending = None
        if defer_final and "start" in outcome:
            pending = {"initial": outcome["initial"], "suppress": outcome["suppress"], "layers": layers,
                       "start": outcome["start"]}
        return result, exported, pending

    def _advance(self, eng: BlockEngine, block: DecoderBlock, inputs, outputs, targets, suppress):
        """The committed block over every batch of ``inputs`` into ``outputs``;
        with ``targets``, the mean score of the outputs against them (the
        arithmetic of ``_scores``)."""
        eng.load_dense(block.weights.linears)
        acc = torch.zeros(len(inputs), dtype=torch.float32, device=eng.device) if targets else None
        for b, (x, out) in enumerate(zip(inputs, outputs)):
            self._forward(eng, x, out)
            if targets:
                acc[b:b + 1].copy_(eng.loss(out, targets[b], suppress=suppress, with_grad=False))
        return float(acc.double().sum().item()) / len(inputs) if targets else None

    def _commit(self, block: DecoderBlock, layer: _Layer) -> QuantizedLayer:
        """Codes (one byte each), scale and zero point for export, and the
        layer's weight replaced by its reconstruction (mround/pipeline/runner.py:760-788)."""
        params = layer.params()
        codes, scale, zp = quantize_codes(layer.weight, params, layer.scheme, eps=self.eps,
                                          init_scale=layer.init_scale, narrow=True)
        recon = fake_quantize(layer.weight, params, layer.scheme, eps=self.eps,
                              init_scale=layer.init_scale,
                              out_dtype=block.weights.linears[layer.name].dtype)
        block.weights.linears[layer.name] = recon
        return QuantizedLayer(codes, scale, zp, layer.scheme)

    # ---------------------------------------------------------------- search --
    def _search_scales(self, eng: BlockEngine, block: DecoderBlock, layers: Mapping[str, _Layer],
                       inputs) -> bool:
        """The v2 scale search for every layer whose scheme asks for it
        (mround/pipeline/runner.py:712-759): one forward per calibration batch
        over the original weights collects each linear input's per-channel sum
        of squares, then each searched layer's grid search runs once."""
        searching = [l for l in layers.values() if l.scheme.scale_init is ScaleInit.SEARCHED]
        if not searching:
            return False
        s = block.shape
        dev = inputs[0].device
        imp = {"x1": torch.zeros(s.hidden, device=dev), "attn": torch.zeros(s.n_heads * s.head_dim, device=dev),
               "x2": torch.zeros(s.hidden, device=dev), "act": torch.zeros(s.intermediate, device=dev)}
        eng.load_dense(block.weights.linears)
        scratch = torch.empty_like(inputs[0])
        seq = self.rows
        for x in inputs:
            for lo, hi in self._pieces(x):
                eng.set_sequences((hi - lo) // seq)
                eng.forward(x[lo:hi], scratch[lo:hi], save=False)
                for t in (eng.x1, eng.attn, eng.x2, eng.act):
                    eng.zero_padding(t)  # token rows only
                K.colsumsq(eng.x1, imp["x1"])
                K.colsumsq(eng.attn, imp["attn"])
                K.colsumsq(eng.x2, imp["x2"])
                K.colsumsq(eng.act, imp["act"])
        source = {"self_attn.q_proj": "x1", "self_attn.k_proj": "x1", "self_attn.v_proj": "x1",
                  "self_attn.o_proj": "attn", "mlp.gate_proj": "x2", "mlp.up_proj": "x2",
                  "mlp.down_proj": "act"}
        for layer in searching:
            rows, cols = layer.weight.shape
            found = search_scales(layer.weight, layer.scheme, importance=imp[source[layer.name]])
            layer.init_scale = found.view(rows, cols // layer.scheme.group_size)
        torch.cuda.synchronize(dev)
        return True

    # ------------------------------------------------------------------ tune --
    def _quantize_all(self, eng: BlockEngine, layers: Mapping[str, _Layer]) -> None:
        """Every tuned layer's W' into the engine's fused operands (in split
        precision as fp32 into ``w32``, then split)."""
        for layer in layers.values():
            p = layer.placement
            K.fq_forward_mapped(layer.weight, layer.v, layer.alpha, layer.beta,
                                bits=layer.scheme.bits, group_size=layer.scheme.group_size,
                                mode=layer.mode, eps=self.eps,
                                wq_out=eng.w32[p.operand] if eng.split else eng.wq[p.operand],
                                row_block=p.row_block, row_stride=p.row_stride,
                                row_offset=p.row_offset, init_scale=layer.init_scale)
        if eng.split:
            eng.split_weights()

    def _step_all(self, eng: BlockEngine, layers: Mapping[str, _Layer], rates: Mapping[str, float],
                  step: int, *, requant: bool = False) -> None:
        """The fused sign-SGD step of every layer; with ``requant`` the same
        kernels also write the new W' into the engine's fused operands (the
        next step's forward, made without rereading W and v; in split
        precision W' is made afterwards in fp32 and split)."""
        if requant and eng.split:
            self._step_all(eng, layers, rates, step)
            self._quantize_all(eng, layers)
            return
        iters = self.tuning.iters
        for name, layer in layers.items():
            p = layer.placement
            lo, hi = layer.scheme.coefficient_bounds
            lr = LinearDecay(rates[name], iters)(step)
            common = dict(bits=layer.scheme.bits, group_size=layer.scheme.group_size, mode=layer.mode,
                          eps=self.eps, lr=lr, coef_lo=lo, coef_hi=hi, v_bound=V_BOUND,
                          row_block=p.row_block, row_stride=p.row_stride, row_offset=p.row_offset,
                          init_scale=layer.init_scale)
            if requant:
                K.fq_step_requant_mapped(layer.weight, layer.v, layer.alpha, layer.beta, eng.dw[p.operand],
                                         wq_out=eng.wq[p.operand], **common)
            else:
                K.fq_step_mapped(layer.weight, layer.v, layer.alpha, layer.beta, eng.dw[p.operand],
                                 **common)

    def _use_graphs(self, eng: BlockEngine, n_batches: int) -> bool:
        """Whether the tuning steps replay a recorded HIP graph per batch: when
        the host's launch latency, not the kernels, bounds a step (a few
        batches of a small block) and no launch is being timed. Each batch's
        graph is recorded once per block and replayed on every later step
        that uses the batch; the rates come from a schedule in device memory
        indexed by a device step counter the graph advances."""
        if eng.capacity * eng.seq_len != self._batch_tokens or eng.split:
            return False  # steps in pieces, and split precision, run from the host
        if self.graphs is not None:
            return bool(self.graphs) and eng.timers is None
        small = eng.tokens * eng.shape.hidden <= GRAPH_MAX_ELEMENTS
        return eng.timers is None and small and n_batches * GRAPH_MIN_REPLAYS <= self.tuning.iters

    def _step_all_scheduled(self, eng: BlockEngine, layers: Mapping[str, _Layer],
                            sched: Mapping[str, torch.Tensor], counter: torch.Tensor) -> None:
        """``_step_all(requant=True)`` with each layer's rate read on the device
        from its schedule at the step counter."""
        for name, layer in layers.items():
            p = layer.placement
            lo, hi = layer.scheme.coefficient_bounds
            K.fq_step_requant_sched(layer.weight, layer.v, layer.alpha, layer.beta, eng.dw[p.operand],
                                    bits=layer.scheme.bits, group_size=layer.scheme.group_size,
                                    mode=layer.mode, eps=self.eps, lr_table=sched[name], step=counter,
                                    coef_lo=lo, coef_hi=hi, v_bound=V_BOUND, row_block=p.row_block,
                                    row_stride=p.row_stride, row_offset=p.row_offset,
                                    wq_out=eng.wq[p.operand], init_scale=layer.init_scale)

    def _gradients(self, eng: BlockEngine, x, target, scratch, suppress: bool, loss_out) -> None:
        """One step's loss (into ``loss_out``) and dL/dW' of every layer (into
        ``eng.dw``) for the batch ``x``. A batch in pieces is still one step
        (mround/pipeline/runner.py:955-1044): each piece's loss is its squared
        errors over the whole batch's element count and the pieces' weight
        gradients are summed; the outlier rule's threshold is first taken over
        the whole batch's output, from a forward pass without activations."""
        pieces = self._pieces(x)
        if len(pieces) == 1:
            eng.set_sequences(eng.capacity)
            eng.forward(x, scratch, save=True)
            loss_out.copy_(eng.loss(scratch, target, suppress=suppress, with_grad=True))
            eng.backward()
            return
        n = eng.real_elements(x)
        threshold = None
        if suppress:
            self._forward(eng, x, scratch)
            eng.loss(scratch, target, suppress=True, with_grad=False)
            threshold = eng.threshold
        loss_out.zero_()
        seq = self.rows
        for i, (lo, hi) in enumerate(pieces):
            eng.set_sequences((hi - lo) // seq)
            eng.forward(x[lo:hi], scratch[lo:hi], save=True)
            loss_out.add_(eng.loss(scratch[lo:hi], target[lo:hi], suppress=suppress, with_grad=True, denom=n,
                                   threshold=threshold))
            eng.backward(accumulate=i > 0)

    def _scores(self, eng, layers, inputs, targets, over, suppress, scratch) -> float:
        """Mean loss over batches ``over`` with the current parameters."""
        self._quantize_all(eng, layers)
        acc = torch.zeros(len(over), dtype=torch.float32, device=eng.device)
        for i, b in enumerate(over):
            self._forward(eng, inputs[b], scratch)
            acc[i:i + 1].copy_(eng.loss(scratch, targets[b], suppress=suppress, with_grad=False))
        return float(acc.double().sum().item()) / len(over)

    def _tune(self, eng: BlockEngine, layers: Mapping[str, _Layer], inputs, targets, *,
              defer_final: bool = False) -> dict:
        """mround/pipeline/runner.py:790-953: the last parameters are kept unless
        the score did not improve."""
        suppress, rates = block_recipe(self.tuning, self.scheme.bits,
                                       {n: l.scheme.bits for n, l in layers.items()},
                                       per_layer=self.per_layer_recipe)
        n_batches = len(inputs)
        self._batch_tokens = inputs[0].shape[0]
        held = min(self.holdout_batches, n_batches - 1)
        tuning_batches = list(range(n_batches - held))
        scoring_batches = list(range(n_batches - held, n_batches)) if held else tuning_batches
        scratch = torch.empty_like(inputs[0])
        stages = {}
        t0 = time.perf_counter()
        initial = self._scores(eng, layers, inputs, targets, scoring_batches, suppress, scratch)
        initial_tuning = (self._scores(eng, layers, inputs, targets, tuning_batches, suppress, scratch)
                          if held else initial)
        stages["score"] = time.perf_counter() - t0
        start = {n: l.snapshot() for n, l in layers.items()}

        t0 = time.perf_counter()
        iters = self.tuning.iters
        step_losses = torch.zeros(iters, dtype=torch.float32, device=eng.device)
        self._quantize_all(eng, layers)
        graphs = self._use_graphs(eng, len(tuning_batches))
        if graphs:
            sched = {n: torch.tensor([LinearDecay(rates[n], iters)(t) for t in range(iters)],
                                     dtype=torch.float32, device=eng.device) for n in layers}
            counter = torch.zeros(1, dtype=torch.int32, device=eng.device)
            captured: dict[int, torch.cuda.CUDAGraph] = {}
        for step in range(iters):
            b = tuning_batches[step % len(tuning_batches)]
            if not graphs or step == 0:
                # (step 0 runs eagerly: it also allocates any library workspace
                # the step needs before a graph records it)
                self._gradients(eng, inputs[b], targets[b], scratch, suppress, step_losses[step:step + 1])
                # the step also writes the next step's W'
                self._step_all(eng, layers, rates, step, requant=True)
                if graphs:
                    counter.fill_(1)
                continue
            g = captured.get(b)
            if g is None:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    eng.forward(inputs[b], scratch, save=True)
                    eng.loss(scratch, targets[b], suppress=suppress, with_grad=True)
                    eng.backward()
                    self._step_all_scheduled(eng, layers, sched, counter)
                    K.counter_add(counter, 1)
                captured[b] = g
            g.replay()
            step_losses[step:step + 1].copy_(eng.loss_val)
        torch.cuda.synchronize(eng.device)
        stages["tune"] = time.perf_counter() - t0
        if defer_final and not held:
            return {"initial": initial, "final": initial, "gap": None, "reverted": False,
                    "losses": step_losses.double().cpu().tolist(), "stages": stages,
                    "suppress": suppress, "start": start}

        t0 = time.perf_counter()
        final = self._scores(eng, layers, inputs, targets, scoring_batches, suppress, scratch)
        final_tuning = (self._scores(eng, layers, inputs, targets, tuning_batches, suppress, scratch)
                        if held else final)
        stages["score"] += time.perf_counter() - t0
        gap = None
        if held:
            gap = (1.0 - final_tuning / initial_tuning) - (1.0 - final / initial)
        losses = step_losses.double().cpu().tolist()
        if final >= initial:
            for n, l in layers.items():
                l.restore(start[n])
            return {"initial": initial, "final": initial, "gap": gap, "reverted": True,
                    "losses": losses, "stages": stages}
        return {"initial": initial, "final": final, "gap": gap, "reverted": False, "losses": losses,
                "stages": stages}


def reconstruction_of(eng: BlockEngine, name: str, rows: int) -> torch.Tensor:
    """A layer's current W' (bf16) out of the engine's fused operand."""
    return unplace(eng.wq[eng.place[name].operand], rows, eng.place[name])
