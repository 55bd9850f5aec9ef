"""One decoder block on the GPU: forward, loss, backward and the fused
per-layer sign-SGD step of the tuning loop.

The block is the mlx-lm Qwen2 / Llama decoder layer the reference runs via
``block_output`` (mround/pipeline/blocks.py:578-606):

    x1 = rmsnorm(x) w_in;  qkv = x1 [Wq; Wk; Wv]^T (+ b);  rope(q, k)
    o = causal GQA attention;  h = x + o Wo^T
    x2 = rmsnorm(h) w_post;  act = silu(x2 Wg^T) * (x2 Wu^T);  out = h + act Wd^T

and its backward is the autodiff the reference takes through it
(mround/pipeline/runner.py:920) down to each layer's dL/dW'.

Layout in HBM, all row-major and allocated once per (batch, seq_len):

* The fake-quantized weights W' are bf16, written by the fake-quant kernel
  straight into fused operands: q, k and v rows stacked into one
  ``[(Hq + 2 Hkv) d, h]`` matrix, and gate/up rows interleaved in blocks of 32
  (rows 64b..64b+31 = gate rows 32b.., rows 64b+32.. = up rows 32b..) so one
  GEMM yields both and its epilogue applies SwiGLU.
* dL/dW' comes out of the weight-gradient GEMMs in the same fused layouts,
  float32, and the fused backward + update kernel reads each layer's rows
  from there.
* Activations: the residual stream and the block output are float32
  ``[T, h]``; GEMM operands (normalized inputs, qkv, attention output,
  SwiGLU output) are bf16.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from mround_amd import kernels as K
from mround_amd.exceptions import ArchitectureError

# The block's linears, in the order the reference walks them
# (sorted(named_modules()), mround/pipeline/blocks.py:654-678).
LAYERS = ("mlp.down_proj", "mlp.gate_proj", "mlp.up_proj", "self_attn.k_proj",
          "self_attn.o_proj", "self_attn.q_proj", "self_attn.v_proj")
QKV = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")
SWIGLU_ROWS = 32  # gate/up interleave period in the fused operand
SEQ_ALIGN = 128  # the attention kernels' query/key tile: rows per sequence are a multiple


def aligned_length(n: int) -> int:
    """Rows per sequence the engine runs for sequences of ``n`` tokens: ``n``
    rounded up to the attention tile. The rows past ``n`` are padding at the
    end of each sequence, which the causal mask keeps out of every real row."""
    return -(-int(n) // SEQ_ALIGN) * SEQ_ALIGN


@dataclass(frozen=True)
class BlockShape:
    """Geometry of a Qwen2 / Llama decoder block."""

    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    intermediate: int
    norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    attn_bias: bool = False
    # RoPE frequency scaling as sorted (key, value) pairs of the config's
    # rope_scaling ("rope_type" plus its parameters); empty: none.
    rope_scaling: tuple = ()

    @property
    def qkv_rows(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim

    def linear_shape(self, name: str) -> tuple[int, int]:
        h, d = self.hidden, self.head_dim
        shapes = {
            "self_attn.q_proj": (self.n_heads * d, h),
            "self_attn.k_proj": (self.n_kv_heads * d, h),
            "self_attn.v_proj": (self.n_kv_heads * d, h),
            "self_attn.o_proj": (h, self.n_heads * d),
            "mlp.gate_proj": (self.intermediate, h),
            "mlp.up_proj": (self.intermediate, h),
            "mlp.down_proj": (h, self.intermediate),
        }
        return shapes[name]

    def validate(self, seq_len: int | None = None) -> None:
        """Raise ``ArchitectureError`` for a geometry the block kernels cannot run."""
        problems = []
        if self.head_dim not in (64, 128):
            problems.append(f"head_dim {self.head_dim} is not 64 or 128")
        if self.n_heads % self.n_kv_heads:
            problems.append(f"{self.n_heads} query heads do not group over {self.n_kv_heads} kv heads")
        if self.hidden % 64 or (self.n_heads * self.head_dim) % 64:
            problems.append("hidden and n_heads * head_dim must be multiples of 64")
        if self.intermediate % 64:
            problems.append(f"intermediate size {self.intermediate} is not a multiple of 64")
        if seq_len is not None and seq_len % 128:
            problems.append(f"sequence length {seq_len} is not a multiple of 128")
        if problems:
            raise ArchitectureError("unsupported block geometry: " + "; ".join(problems))


@dataclass(frozen=True)
class Placement:
    """Where a layer's rows sit in its fused operand: layer row r lands on
    ``(r // row_block) * row_stride + row_offset + r % row_block``."""

    operand: str
    row_block: int
    row_stride: int
    row_offset: int


def placements(shape: BlockShape) -> dict[str, Placement]:
    d = shape.head_dim
    q_rows, kv_rows = shape.n_heads * d, shape.n_kv_heads * d
    return {
        "self_attn.q_proj": Placement("qkv", q_rows, q_rows, 0),
        "self_attn.k_proj": Placement("qkv", kv_rows, kv_rows, q_rows),
        "self_attn.v_proj": Placement("qkv", kv_rows, kv_rows, q_rows + kv_rows),
        "self_attn.o_proj": Placement("o", shape.hidden, shape.hidden, 0),
        "mlp.gate_proj": Placement("gu", SWIGLU_ROWS, 2 * SWIGLU_ROWS, 0),
        "mlp.up_proj": Placement("gu", SWIGLU_ROWS, 2 * SWIGLU_ROWS, SWIGLU_ROWS),
        "mlp.down_proj": Placement("down", shape.hidden, shape.hidden, 0),
    }


def place(fused: torch.Tensor, rows: torch.Tensor, p: Placement) -> None:
    """Copy a layer's rows into its fused operand (host-side layout helper)."""
    n = rows.shape[0]
    if p.row_block == p.row_stride:
        fused[p.row_offset:p.row_offset + n].copy_(rows)
        return
    view = fused.view(-1, p.row_stride, fused.shape[1])[:, p.row_offset:p.row_offset + p.row_block]
    view.copy_(rows.view(-1, p.row_block, rows.shape[1]))


def unplace(fused: torch.Tensor, n: int, p: Placement) -> torch.Tensor:
    """A layer's rows out of its fused operand."""
    if p.row_block == p.row_stride:
        return fused[p.row_offset:p.row_offset + n]
    view = fused.view(-1, p.row_stride, fused.shape[1])[:, p.row_offset:p.row_offset + p.row_block]
    return view.reshape(n, fused.shape[1])


@dataclass
class BlockWeights:
    """A block's parameters on the device: the seven linears ``[out, in]`` in
    the model dtype, the q/k/v biases (float32, when the block has them) and
    the two RMSNorm weights (float32)."""

    linears: dict[str, torch.Tensor]
    biases: dict[str, torch.Tensor] = field(default_factory=dict)
    input_norm: torch.Tensor | None = None
    post_norm: torch.Tensor | None = None

    @classmethod
    def random(cls, shape: BlockShape, *, dtype: torch.dtype, device, seed: int, std: float = 0.02):
        """Random-init weights N(0, std) drawn on ``device`` (norm weights 1, biases N(0, std))."""
        device = torch.device(device)
        g = torch.Generator(device=device).manual_seed(seed)
        lin = {n: (torch.randn(*shape.linear_shape(n), generator=g, device=device) * std).to(dtype)
               for n in LAYERS}
        biases = {}
        if shape.attn_bias:
            biases = {n: torch.randn(shape.linear_shape(n)[0], generator=g, device=device) * std
                      for n in QKV}
        ones = torch.ones(shape.hidden, device=device)
        return cls(lin, biases, ones, ones.clone())


def gemm_problems(shape: BlockShape, tokens: int) -> list[tuple[int, int, int]]:
    """(M, N, K) of every product of a block's forward and backward at
    ``tokens`` tokens (N is the product's width: 2 x intermediate for the
    SwiGLU pair), the shapes whose k-split partials share one workspace."""
    T, h, mlp, q = tokens, shape.hidden, shape.intermediate, shape.qkv_rows
    hq_d = shape.n_heads * shape.head_dim
    return [(T, q, h), (T, h, hq_d), (T, 2 * mlp, h), (T, h, mlp), (T, mlp, h), (h, mlp, T),
            (T, h, 2 * mlp), (2 * mlp, h, T), (T, hq_d, h), (h, hq_d, T), (q, h, T), (T, h, q)]


def split_gemm_problems(shape: BlockShape, tokens: int) -> list[tuple[int, int, int]]:
    """(M, N, K) of the forward products that split precision runs over K' = 3K
    (the q/k/v projection, the attention output projection, the gate/up pair
    and down)."""
    T, h, mlp, q = tokens, shape.hidden, shape.intermediate, shape.qkv_rows
    hq_d = shape.n_heads * shape.head_dim
    return [(T, q, 3 * h), (T, h, 3 * hq_d), (T, 2 * mlp, 3 * h), (T, h, 3 * mlp)]


def workspace_bytes(shape: BlockShape, batch: int, seq_len: int,
                    extra_gemms: tuple[tuple[int, int, int], ...] = (), split: bool = False) -> tuple[int, int]:
    """Bytes of the GEMM k-split workspace (the largest any of the block's
    products, its split-precision products with ``split``, or the caller's
    ``extra_gemms`` plans) and of the attention backward's dK/dV partials (its
    automatic head split) for a block engine of ``batch`` sequences. The
    engine also runs any smaller number of sequences (the pieces of a step,
    ``set_sequences``), whose plans can ask for more (a grid that needs no
    head split at 8 sequences can at 7), so both are the largest over
    1..``batch`` sequences: a piece never runs short of workspace."""
    gemm = max([K.gemm_workspace_bytes(M, N, Kd) for M, N, Kd in extra_gemms], default=0)
    attn = 0
    for n in range(1, batch + 1):
        probs = gemm_problems(shape, n * seq_len) + (split_gemm_problems(shape, n * seq_len) if split else [])
        gemm = max(gemm, max(K.gemm_workspace_bytes(M, N, Kd) for M, N, Kd in probs))
        attn = max(attn, K.attn_bwd_workspace_bytes(batch=n, seq_len=seq_len, n_heads=shape.n_heads,
                                                    n_kv_heads=shape.n_kv_heads, head_dim=shape.head_dim))
    return gemm, attn


ROPE_TYPES = ("default", "linear", "llama3")


def rope_frequencies(head_dim: int, theta: float, scaling: tuple = ()) -> torch.Tensor:
    """The rotary frequencies ``theta^(-2i/d)`` (float64), rescaled as the
    config's ``rope_scaling`` asks: "linear" divides every frequency by
    ``factor``; "llama3" (Meta's Llama 3.1 rule) keeps the frequencies whose
    wavelength is under ``original_max_position_embeddings / high_freq_factor``,
    divides those over ``original_max_position_embeddings / low_freq_factor``
    by ``factor``, and blends the two linearly in between, by where
    ``original_max_position_embeddings / wavelength`` falls between the two
    factors."""
    inv = theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim)
    params = dict(scaling)
    kind = params.get("rope_type", "default")
    if kind == "default":
        return inv
    factor = float(params["factor"])
    if kind == "linear":
        return inv / factor
    if kind == "llama3":
        low, high = float(params["low_freq_factor"]), float(params["high_freq_factor"])
        context = float(params["original_max_position_embeddings"])
        wavelength = 2 * math.pi / inv
        blend = ((context / wavelength - low) / (high - low)).clamp(0.0, 1.0)
        scaled = (1 - blend) * inv / factor + blend * inv
        return torch.where(wavelength < context / high, inv,
                           torch.where(wavelength > context / low, inv / factor, scaled))
    raise ArchitectureError(f"rope_scaling type {kind!r} is not supported (supported: {', '.join(ROPE_TYPES)})")


def rope_table(seq_len: int, head_dim: int, theta: float, device, scaling: tuple = ()) -> torch.Tensor:
    """cos/sin of ``pos * frequency_i``, float32 ``[S, d/2, 2]`` (computed in float64)."""
    inv = rope_frequencies(head_dim, theta, scaling)
    ang = torch.arange(seq_len, dtype=torch.float64)[:, None] * inv[None, :]
    return torch.stack([torch.cos(ang), torch.sin(ang)], -1).float().to(device)


class BlockEngine:
    """Forward, loss and backward of one block over ``batch`` sequences of
    ``seq_len`` rows, with every buffer allocated once.

    ``real_len`` (default ``seq_len``) is how many of a sequence's rows are
    tokens; the rest are padding at its end (``aligned_length``). Causal
    attention keeps padding rows out of every token row, and ``loss`` counts
    token rows only, so the loss and every gradient are those of the
    ``real_len``-token sequences.

    ``split`` runs the forward in split precision (the reference's
    three-product remedy for the block objective, mround DOCUMENTATION.md:
    885-925): the normalized inputs, q/k/v (rotated in fp32), the attention's
    probabilities and output, the SwiGLU output and every W' are carried as
    bf16 hi and lo halves, and each product is three bf16 products (one GEMM
    over K' = 3K of [A_hi | A_hi | A_lo] and [B_hi | B_lo | B_hi]; inside the
    attention, hi hi + lo hi + hi lo). The backward stays in bf16 on the hi
    halves. Weights are written through ``w32`` (fp32) and ``split_weights``."""

    def __init__(self, shape: BlockShape, *, batch: int, seq_len: int, device,
                 extra_gemms: tuple[tuple[int, int, int], ...] = (), real_len: int | None = None,
                 split: bool = False) -> None:
        shape.validate(seq_len)
        self.shape, self.batch, self.seq_len = shape, batch, seq_len
        self.real_len = seq_len if real_len is None else int(real_len)
        if not 1 <= self.real_len <= seq_len:
            raise ArchitectureError(f"{self.real_len} tokens do not fit sequences of {seq_len} rows")
        self.split = bool(split)
        self.device = torch.device(device)
        T, h, mlp = batch * seq_len, shape.hidden, shape.intermediate
        self.tokens = T
        hq_d = shape.n_heads * shape.head_dim
        bf, f32 = torch.bfloat16, torch.float32
        e = lambda *s, dt=bf: torch.empty(*s, dtype=dt, device=self.device)
        # fused W' operands and their gradients
        self.wq = {"qkv": e(shape.qkv_rows, h), "o": e(h, hq_d), "gu": e(2 * mlp, h), "down": e(h, mlp)}
        self.dw = {k: torch.empty(v.shape, dtype=f32, device=self.device) for k, v in self.wq.items()}
        self.bias_qkv = None
        self.norm_in = self.norm_post = None
        # activations
        self.x1, self.rstd1 = e(T, h), e(T, dt=f32)
        self.qkv = e(T, shape.qkv_rows)
        self.attn, self.lse = e(T, hq_d), e(batch, shape.n_heads, seq_len, dt=f32)
        self.h2 = e(T, h, dt=f32)
        self.x2, self.rstd2 = e(T, h), e(T, dt=f32)
        self.act, self.gu = e(T, mlp), e(T, 2 * mlp)
        # backward
        self.grad_out, self.grad_out16 = e(T, h, dt=f32), e(T, h)
        self.dgu = e(T, 2 * mlp)
        self.dx2 = e(T, h, dt=f32)
        self.dh2 = e(T, h)
        self.dattn, self.dsum = e(T, hq_d), e(batch, shape.n_heads, seq_len, dt=f32)
        self.dqkv = e(T, shape.qkv_rows)
        self.loss_val = e(1, dt=f32)
        self.threshold = e(1, dt=f32)
        # split precision: fp32 W' and the split operands
        self.w32 = self.wqs = None
        self.x1s = self.x2s = self.acts = self.gu32 = self.qkv32 = self.qkv_lo = self.attns = None
        if self.split:
            self.w32 = {k: torch.empty(v.shape, dtype=f32, device=self.device) for k, v in self.wq.items()}
            self.wqs = {k: e(v.shape[0], 3 * v.shape[1]) for k, v in self.wq.items()}
            self.x1s, self.x2s = e(T, 3 * h), e(T, 3 * h)
            self.acts, self.gu32 = e(T, 3 * mlp), e(T, 2 * mlp, dt=f32)
            self.qkv32, self.qkv_lo = e(T, shape.qkv_rows, dt=f32), e(T, shape.qkv_rows)
            self.attns = e(T, 3 * hq_d)
        self.cos_sin = rope_table(seq_len, shape.head_dim, shape.rope_theta, self.device, shape.rope_scaling)
        self.scale = 1.0 / math.sqrt(shape.head_dim)
        self.place = placements(shape)
        self.loss_ws = K.loss_workspace(self.device, T * h)
        # the library's scratch for the GEMM k-split partials and the attention
        # backward's dK/dV partials, owned here (extra_gemms: products a caller
        # runs with this workspace besides the block's own)
        gemm_b, attn_b = workspace_bytes(shape, batch, seq_len, extra_gemms, self.split)
        self.gemm_ws = e(gemm_b, dt=torch.uint8) if gemm_b else None
        self.attn_ws = e(attn_b, dt=torch.uint8) if attn_b else None
        self.x_in: torch.Tensor | None = None  # block input of the last saving forward
        self.dh32: torch.Tensor | None = None  # fp32 residual gradient, for input gradients
        self.capacity = batch  # sequences the buffers hold (see set_sequences)
        self._per_token = self.PER_TOKEN + (self.SPLIT_PER_TOKEN if self.split else ())
        self._full = {n: getattr(self, n) for n in self._per_token + self.PER_SEQUENCE}
        # name -> [(start, end) HIP events] for the launches being timed, or None
        self.timers: dict[str, list] | None = None

    # What a forward(save=True) leaves for the backward, besides its input.
    ACTIVATIONS = ("x1", "rstd1", "qkv", "attn", "lse", "h2", "x2", "rstd2", "act", "gu")
    # Buffers with a row per token, and with a leading sequence dimension.
    PER_TOKEN = ("x1", "rstd1", "qkv", "attn", "h2", "x2", "rstd2", "act", "gu", "grad_out",
                 "grad_out16", "dgu", "dx2", "dh2", "dattn", "dqkv")
    PER_SEQUENCE = ("lse", "dsum")
    SPLIT_PER_TOKEN = ("x1s", "x2s", "acts", "gu32", "qkv32", "qkv_lo", "attns")

    def set_sequences(self, n: int) -> None:
        """Run the next passes over ``n`` sequences (at most the capacity the
        engine was built for): every per-token buffer becomes a view of its
        first ``n * seq_len`` rows. A step's batch runs in pieces this way
        (``TuningConfig.micro_batches``) on one set of buffers."""
        if not 1 <= n <= self.capacity:
            raise ArchitectureError(f"{n} sequences do not fit an engine built for {self.capacity}")
        if n == self.batch:
            return
        T = n * self.seq_len
        for name in self._per_token:
            setattr(self, name, self._full[name][:T])
        for name in self.PER_SEQUENCE:
            setattr(self, name, self._full[name][:n])
        self.batch, self.tokens = n, T

    def new_activations(self) -> dict[str, torch.Tensor]:
        """A fresh set of the saved-activation buffers, for keeping several
        blocks' activations at once (see ``bind``)."""
        return {n: torch.empty_like(getattr(self, n)) for n in self.ACTIVATIONS}

    def bind(self, acts: dict[str, torch.Tensor], x_in: torch.Tensor | None = None) -> None:
        """Make ``acts`` the saved-activation buffers that the next forward
        writes and the next backward reads, and ``x_in`` the block input that
        they were saved from (kept unchanged by the caller)."""
        for n in self.ACTIVATIONS:
            setattr(self, n, acts[n])
        self.x_in = x_in

    def _run(self, name: str, fn) -> None:
        """Launch ``fn``; bracket it with events on the current stream when timed."""
        if self.timers is None or name not in self.timers:
            fn()
            return
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        self.timers[name].append((start, end))

    def time_launches(self, names) -> None:
        """Start recording HIP events around the named launches (see ``flops``)."""
        self.timers = {n: [] for n in names}

    def launch_ms(self) -> dict[str, list[float]]:
        """Recorded durations per launch name (synchronizes)."""
        torch.cuda.synchronize(self.device)
        return {n: [s.elapsed_time(e) for s, e in ev] for n, ev in (self.timers or {}).items()}

    def flops(self) -> dict[str, float]:
        """Algorithmic flops of one launch of each timed operation (2 M N K for a
        GEMM; attention counts the causal half of QK^T and PV, 2.5x that backward)."""
        s, T = self.shape, self.tokens
        h, hq_d, mlp, q = s.hidden, s.n_heads * s.head_dim, s.intermediate, s.qkv_rows
        attn = 4.0 * self.batch * self.seq_len * self.seq_len * s.n_heads * s.head_dim / 2
        return {
            "gemm_qkv": 2.0 * T * q * h, "gemm_o": 2.0 * T * h * hq_d,
            "gemm_gate_up": 2.0 * T * 2 * mlp * h, "gemm_down": 2.0 * T * h * mlp,
            "attn_fwd": attn, "attn_bwd": 2.5 * attn,
            "gemm_dact": 2.0 * T * mlp * h, "gemm_dw_down": 2.0 * h * mlp * T,
            "gemm_dx_gate_up": 2.0 * T * h * 2 * mlp, "gemm_dw_gate_up": 2.0 * 2 * mlp * h * T,
            "gemm_dattn": 2.0 * T * hq_d * h, "gemm_dw_o": 2.0 * h * hq_d * T,
            "gemm_dw_qkv": 2.0 * q * h * T, "gemm_dx_qkv": 2.0 * T * h * q,
        }

    # ---------------------------------------------------------------- weights --
    def set_block(self, weights: BlockWeights) -> None:
        """Biases and norm weights of the block (kept fp32)."""
        s = self.shape
        if s.attn_bias:
            if set(weights.biases) != set(QKV):
                raise ArchitectureError("the block geometry has q/k/v biases but the weights do not")
            self.bias_qkv = torch.cat([weights.biases[n].float() for n in QKV]).contiguous()
        else:
            self.bias_qkv = None
        self.norm_in = weights.input_norm.float().contiguous()
        self.norm_post = weights.post_norm.float().contiguous()

    def load_dense(self, linears: dict[str, torch.Tensor]) -> None:
        """W' = the given weights rounded to bf16 (the targets pass, and the
        advance pass over committed reconstructions); in split precision the
        weights as they are (hi and lo halves, lo zero for bf16 weights)."""
        if self.split:
            for name, p in self.place.items():
                place(self.w32[p.operand], linears[name].float(), p)
            self.split_weights()
            return
        for name, p in self.place.items():
            place(self.wq[p.operand], linears[name].to(torch.bfloat16), p)

    def split_weights(self) -> None:
        """Split precision: every fused fp32 W' in ``w32`` into its split
        operand, and its hi half into ``wq`` (what the backward reads)."""
        for k, w in self.w32.items():
            K.split_bf16(w, self.wqs[k], order=K.SPLIT_WEIGHT, plain=self.wq[k])

    # ---------------------------------------------------------------- forward --
    def forward(self, x: torch.Tensor, out: torch.Tensor, *, save: bool) -> None:
        """``out = block(x)``; ``x``/``out`` float32 ``[T, h]`` (``out`` may be ``x``).
        ``save`` keeps what the backward reads."""
        s, T = self.shape, self.tokens
        if x.shape != (T, s.hidden) or out.shape != (T, s.hidden):
            raise ArchitectureError(f"block input must be [{T}, {s.hidden}]")
        h, hq_d, mlp = s.hidden, s.n_heads * s.head_dim, s.intermediate
        ws = self.gemm_ws
        if save:
            if out.data_ptr() == x.data_ptr():
                raise ArchitectureError("a saving forward needs its input kept: out must not be x")
            self.x_in = x
        if self.split:
            self._forward_split(x, out)
            return
        K.rmsnorm_fwd(x, self.norm_in, s.norm_eps, self.x1, self.rstd1)
        self._run("gemm_qkv", lambda: K.gemm("nt", self.x1, self.wq["qkv"], self.qkv, M=T, N=s.qkv_rows,
                                             K=h, bias=self.bias_qkv, workspace=ws))
        K.rope(self.qkv, seq_len=self.seq_len, n_heads=s.n_heads + s.n_kv_heads, head_dim=s.head_dim,
               cos_sin=self.cos_sin)
        self._run("attn_fwd", lambda: K.attn_fwd(
            self.qkv, batch=self.batch, seq_len=self.seq_len, n_heads=s.n_heads,
            n_kv_heads=s.n_kv_heads, head_dim=s.head_dim, scale=self.scale, out=self.attn, lse=self.lse))
        self._run("gemm_o", lambda: K.gemm("nt", self.attn, self.wq["o"], self.h2, M=T, N=h, K=hq_d,
                                           resid=x, workspace=ws))
        K.rmsnorm_fwd(self.h2, self.norm_post, s.norm_eps, self.x2, self.rstd2)
        self._run("gemm_gate_up", lambda: K.gemm_swiglu(self.x2, self.wq["gu"], self.act,
                                                        self.gu if save else None, workspace=ws))
        self._run("gemm_down", lambda: K.gemm("nt", self.act, self.wq["down"], out, M=T, N=h, K=mlp,
                                              resid=self.h2, workspace=ws))

    def _forward_split(self, x: torch.Tensor, out: torch.Tensor) -> None:
        """``forward`` with the products in split precision (see the class);
        leaves the same saved activations (x1, x2 and act as their hi halves)."""
        s, T = self.shape, self.tokens
        h, hq_d, mlp = s.hidden, s.n_heads * s.head_dim, s.intermediate
        ws = self.gemm_ws
        K.rmsnorm_fwd_split(x, self.norm_in, s.norm_eps, self.x1s, self.x1, self.rstd1)
        self._run("gemm_qkv", lambda: K.gemm("nt", self.x1s, self.wqs["qkv"], self.qkv32, M=T, N=s.qkv_rows,
                                             K=3 * h, bias=self.bias_qkv, workspace=ws))
        # rotated in fp32, then hi (the backward's q/k/v) and lo halves
        K.rope_split(self.qkv32, self.qkv, self.qkv_lo, seq_len=self.seq_len,
                     n_rope_heads=s.n_heads + s.n_kv_heads, head_dim=s.head_dim, cos_sin=self.cos_sin)
        self._run("attn_fwd", lambda: K.attn_fwd_split(
            self.qkv, self.qkv_lo, batch=self.batch, seq_len=self.seq_len, n_heads=s.n_heads,
            n_kv_heads=s.n_kv_heads, head_dim=s.head_dim, scale=self.scale, out=self.attn,
            out_split=self.attns, lse=self.lse))
        self._run("gemm_o", lambda: K.gemm("nt", self.attns, self.wqs["o"], self.h2, M=T, N=h, K=3 * hq_d,
                                           resid=x, workspace=ws))
        K.rmsnorm_fwd_split(self.h2, self.norm_post, s.norm_eps, self.x2s, self.x2, self.rstd2)

        def gate_up():
            K.gemm("nt", self.x2s, self.wqs["gu"], self.gu32, M=T, N=2 * mlp, K=3 * h, workspace=ws)
            K.swiglu_split(self.gu32, self.acts, self.act, self.gu)
        self._run("gemm_gate_up", gate_up)
        self._run("gemm_down", lambda: K.gemm("nt", self.acts, self.wqs["down"], out, M=T, N=h, K=3 * mlp,
                                              resid=self.h2, workspace=ws))

    def loss(self, out: torch.Tensor, target: torch.Tensor, *, suppress: bool, with_grad: bool,
             denom: int | None = None, threshold: torch.Tensor | None = None) -> torch.Tensor:
        """Reconstruction loss of one batch (device scalar), and dL/dout when asked:
        mean squared error, or with the top 0.1 % of |residuals| excluded
        (mround/core/losses.py:42-107). A piece of a batch passes the whole
        batch's element count (``real_elements``) as ``denom`` and, with the
        outlier rule, the whole batch's ``threshold`` (``piece_loss``,
        mround/core/losses.py:110-130). With padded sequences the padding rows
        of ``out`` take ``target``'s values first: their residuals are zero,
        so they add nothing to the loss or its gradient and, lying below every
        kept magnitude, leave the k-th largest |residual| unchanged."""
        if self.real_len < self.seq_len:
            S, r = self.seq_len, self.real_len
            n_seq = out.shape[0] // S
            out.view(n_seq, S, -1)[:, r:].copy_(target.view(n_seq, S, -1)[:, r:])
        n = self.real_elements(out)
        denom = n if denom is None else denom
        grad = self.grad_out if with_grad else None
        if suppress and threshold is not None:
            K.loss_outlier(out, target, k=1, denom=denom, loss_out=self.loss_val, threshold_in=threshold,
                           grad_out=grad, workspace=self.loss_ws)
        elif suppress:
            K.loss_outlier(out, target, k=max(1, int(n * 0.001)), denom=denom, loss_out=self.loss_val,
                           threshold_out=self.threshold, grad_out=grad, workspace=self.loss_ws)
        else:
            K.loss_mse(out, target, denom=denom, loss_out=self.loss_val, grad_out=grad,
                       workspace=self.loss_ws)
        return self.loss_val

    def real_elements(self, t: torch.Tensor) -> int:
        """Elements of the token rows of ``t`` (whole sequences of ``seq_len`` rows)."""
        return t.numel() // self.seq_len * self.real_len

    def zero_padding(self, t: torch.Tensor) -> None:
        """Clear the padding rows of ``t`` (whole sequences of ``seq_len`` rows)."""
        if self.real_len < self.seq_len:
            t.view(t.shape[0] // self.seq_len, self.seq_len, -1)[:, self.real_len:].zero_()

    # --------------------------------------------------------------- backward --
    def backward(self, dx_out: torch.Tensor | None = None, *, accumulate: bool = False) -> None:
        """dL/dW' of all seven layers into ``self.dw`` from ``self.grad_out``
        (after ``forward(save=True)`` and ``loss(with_grad=True)``, or with
        ``grad_out`` filled by the caller); ``accumulate`` adds them to what
        ``self.dw`` holds (the weight-gradient products' residual epilogue), as
        the pieces of a batch do. With ``dx_out`` (float32 ``[T, h]``, not
        ``grad_out``) also the gradient with respect to the block input."""
        s, T = self.shape, self.tokens
        if dx_out is not None:
            if self.x_in is None:
                raise ArchitectureError("the input gradient needs a saving forward first")
            if dx_out.shape != (T, s.hidden) or dx_out.dtype != torch.float32:
                raise ArchitectureError(f"dx_out must be float32 [{T}, {s.hidden}]")
            if dx_out.data_ptr() == self.grad_out.data_ptr():
                raise ArchitectureError("dx_out must not be the output gradient buffer")
            if self.dh32 is None or self.dh32.shape[0] != T:
                self.dh32 = torch.empty(T, s.hidden, dtype=torch.float32, device=self.device)
        h, hq_d, mlp = s.hidden, s.n_heads * s.head_dim, s.intermediate
        ws = self.gemm_ws
        acc = (lambda k: self.dw[k]) if accumulate else (lambda k: None)
        K.cast_bf16(self.grad_out, self.grad_out16)
        # MLP: dgu from dact = dout Wd'; dWd' = dout^T act; dx2 = dgu Wgu'; dWgu' = dgu^T x2
        self._run("gemm_dact", lambda: K.gemm_swiglu_bwd(self.grad_out16, self.wq["down"], self.gu,
                                                         self.dgu, workspace=ws))
        self._run("gemm_dw_down", lambda: K.gemm("tn", self.grad_out16, self.act, self.dw["down"], M=h,
                                                 N=mlp, K=T, resid=acc("down"), workspace=ws))
        self._run("gemm_dx_gate_up", lambda: K.gemm("nn", self.dgu, self.wq["gu"], self.dx2, M=T, N=h,
                                                    K=2 * mlp, workspace=ws))
        self._run("gemm_dw_gate_up", lambda: K.gemm("tn", self.dgu, self.x2, self.dw["gu"], M=2 * mlp,
                                                    N=h, K=T, resid=acc("gu"), workspace=ws))
        # dh = dout + rmsnorm'(dx2)
        K.rmsnorm_bwd(self.dx2, self.h2, self.norm_post, self.rstd2, self.grad_out, dh_bf16=self.dh2,
                      dh_f32=self.dh32 if dx_out is not None else None)
        # attention output projection
        self._run("gemm_dattn", lambda: K.gemm("nn", self.dh2, self.wq["o"], self.dattn, M=T, N=hq_d,
                                               K=h, workspace=ws))
        self._run("gemm_dw_o", lambda: K.gemm("tn", self.dh2, self.attn, self.dw["o"], M=h, N=hq_d,
                                              K=T, resid=acc("o"), workspace=ws))
        self._run("attn_bwd", lambda: K.attn_bwd(
            self.qkv, self.attn, self.dattn, self.lse, self.dsum, batch=self.batch,
            seq_len=self.seq_len, n_heads=s.n_heads, n_kv_heads=s.n_kv_heads, head_dim=s.head_dim,
            scale=self.scale, dqkv=self.dqkv, workspace=self.attn_ws))
        K.rope(self.dqkv, seq_len=self.seq_len, n_heads=s.n_heads + s.n_kv_heads,
               head_dim=s.head_dim, cos_sin=self.cos_sin, backward=True)
        self._run("gemm_dw_qkv", lambda: K.gemm("tn", self.dqkv, self.x1, self.dw["qkv"], M=s.qkv_rows,
                                                N=h, K=T, resid=acc("qkv"), workspace=ws))
        if dx_out is None:
            return
        # dx = dh + rmsnorm'(dqkv Wqkv'); dx2 is free again and holds dx1.
        self._run("gemm_dx_qkv", lambda: K.gemm("nn", self.dqkv, self.wq["qkv"], self.dx2, M=T, N=h,
                                                K=s.qkv_rows, workspace=ws))
        K.rmsnorm_bwd(self.dx2, self.x_in, self.norm_in, self.rstd1, self.dh32, dh_f32=dx_out)
