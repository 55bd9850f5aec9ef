"""Peak device memory of a run, predicted from the model's configuration
alone (the role of mround/planner/memory.py:458-760 and ``predict_memory``,
mround/api.py:1088-1192, on one MI355X).

The reference's rule is a fit to measured MLX runs on unified memory. Here the
run allocates every buffer itself, so the prediction is an account of them,
stage by stage:

* ``load``: the model on the device (block linears and embeddings in the
  model dtype, norms and q/k/v biases widened to fp32);
* ``scoring`` (mixed runs without a given plan): the causal-LM engine of the
  scoring pass (``mround_amd.pipeline.causal_lm``): a fused bf16 copy of every
  block's W', every block's saved activations, the residual stream at each
  block boundary, the logits and the block engine at the scoring batch;
* ``blocks``: the calibration token ids, the fp32 calibration streams (with
  quantized inputs the reference and quantized streams, plus the spare the
  advance writes into when no batches are held out and the model is not
  float16; without, the inputs and the targets),
  the block engine at the tuning batch (at its largest piece when steps run
  in pieces), one block's learnables and their snapshot, and the committed
  codes of every block (their peak, at the last block);
* ``remainder``: the round-to-nearest codes of the tensors outside the blocks.

Every block engine holds its own workspaces for the library: the GEMM
k-split partials and the attention backward's dK/dV partials, at the sizes
the library's queries give for the engine's products (the library allocates
nothing itself). Figures are bytes; the torch allocator's rounding adds
under 1 %.
"""

from __future__ import annotations

import dataclasses
from collections.abc import Mapping
from typing import Any

from mround_amd.exceptions import ArchitectureError, MemoryBudgetError

GIB = 1 << 30
LOSS_WORKSPACE = 4_778_016  # mr_loss_workspace_bytes
SEQ_ALIGN = 128  # block.SEQ_ALIGN (this module imports no torch at load time)
_DTYPE_BYTES = {"bfloat16": 2, "float16": 2, "float32": 4}


def _gb(n: float) -> str:
    return f"{n / 1e9:.2f} GB"


@dataclasses.dataclass(frozen=True)
class ModelShape:
    """What the prediction reads from ``config.json``."""

    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    tied: bool
    attn_bias: bool
    dtype_bytes: int = 2

    @classmethod
    def from_config(cls, config: Mapping[str, Any]) -> ModelShape:
        try:
            heads = int(config["num_attention_heads"])
            hidden = int(config["hidden_size"])
            return cls(hidden=hidden, layers=int(config["num_hidden_layers"]), heads=heads,
                       kv_heads=int(config.get("num_key_value_heads") or heads),
                       head_dim=int(config.get("head_dim") or hidden // heads),
                       intermediate=int(config["intermediate_size"]), vocab=int(config["vocab_size"]),
                       tied=bool(config.get("tie_word_embeddings", False)),
                       attn_bias=config.get("model_type") == "qwen2" or bool(config.get("attention_bias")),
                       dtype_bytes=_DTYPE_BYTES.get(str(config.get("torch_dtype", "bfloat16")), 2))
        except (KeyError, TypeError, ValueError) as exc:
            raise ArchitectureError(f"the configuration does not describe a dense decoder: {exc}") from exc

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def layer_shapes(self) -> list[tuple[int, int]]:
        """(out, in) of the seven block linears."""
        h, d = self.hidden, self.head_dim
        return [(self.heads * d, h), (self.kv_heads * d, h), (self.kv_heads * d, h), (h, self.heads * d),
                (self.intermediate, h), (self.intermediate, h), (h, self.intermediate)]

    @property
    def block_weights(self) -> int:
        return sum(o * i for o, i in self.layer_shapes())

    @property
    def largest_layer(self) -> int:
        return max(o * i for o, i in self.layer_shapes())

    def model_bytes(self) -> int:
        """The model as loaded: linears and embeddings in the model dtype, norms
        and biases in fp32."""
        per_block = self.block_weights * self.dtype_bytes + 2 * self.hidden * 4
        if self.attn_bias:
            per_block += self.qkv_rows * 4
        embed = self.vocab * self.hidden * self.dtype_bytes
        head = 0 if self.tied else embed
        return self.layers * per_block + embed + head + self.hidden * self.dtype_bytes


def library_workspace_bytes(m: ModelShape, tokens: int, seq_len: int,
                            extra_gemms: tuple[tuple[int, int, int], ...] = (), split: bool = False) -> int:
    """The GEMM k-split and attention dK/dV workspaces a ``BlockEngine`` at
    ``tokens`` tokens owns (the library's size queries)."""
    from mround_amd.pipeline.block import BlockShape, workspace_bytes

    shape = BlockShape(hidden=m.hidden, n_heads=m.heads, n_kv_heads=m.kv_heads, head_dim=m.head_dim,
                       intermediate=m.intermediate)
    return sum(workspace_bytes(shape, tokens // seq_len, seq_len, extra_gemms, split))


def split_bytes(m: ModelShape, tokens: int) -> int:
    """What split precision adds to a ``BlockEngine``: fp32 W' and the split
    W' operands, the split normalized inputs and SwiGLU output, the fp32
    gate/up pair, the fp32 q/k/v and their lo halves, and the split attention
    output."""
    T, h, mlp, q = tokens, m.hidden, m.intermediate, m.qkv_rows
    hq_d = m.heads * m.head_dim
    return (m.block_weights * (4 + 6) + 2 * T * 3 * h * 2 + T * 3 * mlp * 2 + T * 2 * mlp * 4
            + T * q * (4 + 2) + T * 3 * hq_d * 2)


def engine_bytes(m: ModelShape, tokens: int, seq_len: int, *, input_grads: bool = False,
                 extra_gemms: tuple[tuple[int, int, int], ...] = (), split: bool = False) -> int:
    """``BlockEngine`` at ``tokens`` tokens: fused W' (bf16) and dL/dW' (fp32),
    the saved activations, the backward's buffers and the library workspaces
    (and with ``split``, the split-precision operands)."""
    T, h, q, mlp = tokens, m.hidden, m.qkv_rows, m.intermediate
    hq_d = m.heads * m.head_dim
    weights = m.block_weights * (2 + 4)
    acts = activation_bytes(m, tokens)
    bwd = T * h * 4 + T * h * 2 + T * 2 * mlp * 2 + T * h * 4 + T * h * 2 + T * hq_d * 2 + T * m.heads * 4 + T * q * 2
    rope = seq_len * (m.head_dim // 2) * 2 * 4
    extra = T * h * 4 if input_grads else 0
    scalars = 2 * 4  # loss value and outlier threshold
    ws = library_workspace_bytes(m, tokens, seq_len, extra_gemms, split)
    return (weights + acts + bwd + rope + LOSS_WORKSPACE + scalars + extra + ws
            + (split_bytes(m, tokens) if split else 0))


def activation_bytes(m: ModelShape, tokens: int) -> int:
    """One block's saved activations (``BlockEngine.ACTIVATIONS``)."""
    T, h, mlp = tokens, m.hidden, m.intermediate
    hq_d = m.heads * m.head_dim
    return (T * h * 2 + T * 4 + T * m.qkv_rows * 2 + T * hq_d * 2 + T * m.heads * 4 + T * h * 4 + T * h * 2
            + T * 4 + T * mlp * 2 + T * 2 * mlp * 2)


@dataclasses.dataclass(frozen=True)
class RunShape:
    """The run options the prediction depends on."""

    n_samples: int
    seq_len: int
    batch_size: int
    group_size: int
    searched: bool = False
    quantized_inputs: bool = True
    mixed: bool = False
    widths: int = 1
    gradient_source: str = "own_width"
    scoring_samples: int = 128
    scoring_seq_len: int = 1024
    scoring_batch: int = 2
    dense_remainder: bool = False
    holdout_batches: int = 0
    micro_batches: int = 1
    half: bool = False  # float16 model: the final score is taken apart from the advance
    split: bool = False  # split-precision products (the final score apart from the advance too)

    @property
    def streams(self) -> int:
        """Calibration streams the block loop holds at once."""
        fused = self.quantized_inputs and self.holdout_batches == 0 and not self.half and not self.split
        return 3 if fused else 2

    @property
    def piece_sequences(self) -> int:
        """Sequences the block engine holds: the batch's largest piece."""
        return -(-self.batch_size // max(1, min(self.micro_batches, self.batch_size)))


@dataclasses.dataclass(frozen=True)
class MemoryPrediction:
    """Bytes per stage; ``peak`` is the largest."""

    stages: dict[str, int]

    @property
    def peak(self) -> int:
        return max(self.stages.values())

    @property
    def stage(self) -> str:
        return max(self.stages, key=self.stages.get)

    def record(self) -> dict[str, Any]:
        return {"stages": dict(self.stages), "peak": self.peak, "peak_stage": self.stage}


def aligned_rows(n: int) -> int:
    """Rows per sequence of ``n`` positions (``block.aligned_length``)."""
    return -(-n // SEQ_ALIGN) * SEQ_ALIGN


def _groups(m: ModelShape, gs: int) -> int:
    return sum(o * (i // gs if gs > 0 else 1) for o, i in m.layer_shapes())


def predict_memory(m: ModelShape, run: RunShape) -> MemoryPrediction:
    """Device bytes of each stage of the run (see the module docstring)."""
    base = m.model_bytes()
    stages = {"load": base}
    L, h = m.layers, m.hidden
    if run.mixed:
        S = aligned_rows(run.scoring_seq_len - 1)
        T = run.scoring_batch * S
        Vp = -(-m.vocab // 64) * 64
        lm = (engine_bytes(m, T, S, input_grads=True, extra_gemms=((T, Vp, h), (T, h, Vp)))
              + L * m.block_weights * 2 + L * activation_bytes(m, T)
              + (L + 1 + 2) * T * h * 4 + T * Vp * 2 + T * h * (2 + 4) + T * 4 * 2 + 2 * T * 4 + h * 4 + 4)
        if Vp != m.vocab:
            lm += Vp * h * 2
        grids = 0
        if run.searched:
            per_width = L * _groups(m, run.group_size) * 4
            grids = per_width * (run.widths if run.gradient_source == "widest" else 1)
        tokens = run.scoring_samples * run.scoring_seq_len * 8
        stages["scoring"] = base + lm + grids + tokens + run.n_samples * run.seq_len * 8
    S = aligned_rows(run.seq_len)  # rows per sequence in the streams and the engine
    T = run.batch_size * S
    streams = run.streams * run.n_samples * S * h * 4
    groups = _groups(m, run.group_size)
    learn = m.block_weights * 4 * 2 + groups * 4 * 4 + (groups * 4 if run.searched else 0)
    committed = L * (m.block_weights + groups * 8)
    transient = m.largest_layer * (1 + 4) + T * h * 4
    piece = run.piece_sequences * S
    stages["blocks"] = (base + run.n_samples * run.seq_len * 8 + streams
                        + engine_bytes(m, piece, S, split=run.split)
                        + learn + committed + transient)
    rem = 0
    if not run.dense_remainder:
        rows = m.vocab * (1 if m.tied else 2)
        rem = rows * h + rows * (h // run.group_size if run.group_size > 0 else 1) * 8
    stages["remainder"] = base + committed + rem
    return MemoryPrediction(stages)


@dataclasses.dataclass(frozen=True)
class MemoryCheck:
    """A prediction against a budget (``None``: no budget known)."""

    prediction: MemoryPrediction
    budget: int | None

    @property
    def fits(self) -> bool:
        return self.budget is None or self.prediction.peak <= self.budget

    def describe(self) -> str:
        p = self.prediction
        against = "no budget" if self.budget is None else f"a budget of {_gb(self.budget)}"
        return (f"predicted peak {_gb(p.peak)} in the {p.stage} stage against {against}: "
                + ", ".join(f"{k} {_gb(v)}" for k, v in p.stages.items()))

    def explain(self) -> str:
        if self.fits:
            return self.describe()
        return (self.describe() + ". The calibration streams take 4 bytes per token and hidden unit, "
                "three times with quantized inputs and twice without (or with held-out batches), so fewer "
                "calibration samples, shorter sequences or quantized_inputs=False reduce the blocks stage, "
                "and micro_batches shrinks the step's activations; a smaller scoring_batch_size or "
                "scoring_seq_len reduces the scoring stage")

    def record(self) -> dict[str, Any]:
        return {**self.prediction.record(), "budget": self.budget, "fits": self.fits}


def default_budget(device=None) -> int | None:
    """90 % of the device's memory, or None where no device is visible."""
    try:
        import torch

        if not torch.cuda.is_available():
            return None
        _, total = torch.cuda.mem_get_info(device)
        return int(total * 0.9)
    except Exception:
        return None


def check_memory(m: ModelShape, run: RunShape, *, budget: int | None) -> MemoryCheck:
    """The prediction against ``budget``; raises ``ValueError`` for a budget
    that is not a positive number of bytes."""
    if budget is not None and int(budget) <= 0:
        raise ValueError(f"memory_budget must be a positive number of bytes, got {budget}")
    return MemoryCheck(predict_memory(m, run), None if budget is None else int(budget))


def require_fits(check: MemoryCheck) -> None:
    if not check.fits:
        raise MemoryBudgetError(check.explain())
