"""Whole-model causal-LM loss and the gradient at every block linear, on the GPU.

The mixed-precision scoring pass (mround/pipeline/scoring.py:425-583) takes,
per calibration batch, the gradient of the mean shifted cross-entropy
(``_causal_loss``, scoring.py:183-192) with respect to each block linear's
weight, with every block linear replaced by its quantize-dequantize
(scoring.py:507-514). This module runs that forward and backward through the
block kernels:

    x_0 = embed[ids]                                  mr_embed_rows
    x_{i+1} = block_i(x_i)                            BlockEngine.forward
    logits = rmsnorm(x_L) head^T  (bf16)              mr_rmsnorm_fwd, mr_gemm nt
    loss = mean_t CE(logits_t, label_t)               mr_cross_entropy
    dlogits -> dx_L -> block backward i = L-1 .. 0    mr_gemm nn, mr_rmsnorm_bwd,
                                                      BlockEngine.backward(dx_out)

handing each block's dL/dW' (fused operand layout, fp32) to a callback as soon
as its backward ends, the order the reference accumulates scores in
(scoring.py:238-266).

Sequences of ``seq_len`` tokens feed ``seq_len - 1`` inputs and labels. The
attention kernels need the sequence padded to a multiple of 128: padded
positions come after every real one, so causal attention keeps them out of
every real position, and their labels are ignored, so they contribute exactly
zero to the loss and to every gradient. Batches with fewer sequences than the
engine holds are padded the same way with whole ignored sequences.

Layout in HBM, allocated once:

* ``stream[i]``: float32 ``[T, h]`` input of block i (``stream[L]`` the last
  block's output);
* per block, its fused W' operands (bf16) and, when activations are kept, its
  saved activations (otherwise each block's forward is recomputed before its
  backward, the reference's gradient checkpointing, blocks.py:263-281);
* the head: normalized final hidden state bf16 ``[T, h]``, logits bf16
  ``[T, Vp]`` (Vp = V rounded up to 64) overwritten in place by their gradient,
  and a bf16 head matrix ``[Vp, h]`` whose zero rows past V make the padded
  logits columns zero, so the input-gradient GEMM may run over all Vp.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping

import torch

from mround_amd import kernels as K
from mround_amd.core.quantizer import mode_of
from mround_amd.exceptions import ArchitectureError, CalibrationError
from mround_amd.pipeline.block import LAYERS, BlockEngine, aligned_length, place, placements
from mround_amd.schemes import DEFAULT_EPS_FP32, QuantScheme


def padded_length(seq_len: int) -> int:
    """Positions the engine runs for sequences of ``seq_len`` tokens."""
    return aligned_length(seq_len - 1)


class CausalLM:
    """Loss and block-linear gradients of a ``DecoderModel`` over batches of
    up to ``batch`` token sequences of ``seq_len`` tokens."""

    def __init__(self, model, *, batch: int, seq_len: int, device,
                 keep_activations: bool | None = None) -> None:
        if seq_len < 2:
            raise CalibrationError(f"scoring sequences need at least 2 tokens, got {seq_len}")
        if batch < 1:
            raise CalibrationError(f"scoring batch must hold at least one sequence, got {batch}")
        if not model.blocks:
            raise ArchitectureError("the model has no blocks")
        self.model = model
        self.device = torch.device(device)
        self.shape = model.blocks[0].shape
        for b in model.blocks:
            if b.shape != self.shape:
                raise ArchitectureError("every block must share one geometry")
        self.batch, self.seq_len = batch, seq_len
        self.n_in = seq_len - 1
        S = padded_length(seq_len)
        head = model.embed if model.lm_head is None else model.lm_head
        Vp = -(-int(head.shape[0]) // 64) * 64
        T0, h0 = batch * S, self.shape.hidden
        # the head's two products share the block engine's k-split workspace
        self.eng = BlockEngine(self.shape, batch=batch, seq_len=S, device=self.device,
                               extra_gemms=((T0, Vp, h0), (T0, h0, Vp)))
        eng, T, h = self.eng, self.eng.tokens, self.shape.hidden
        self.tokens = T
        f32, bf = torch.float32, torch.bfloat16
        L = len(model.blocks)
        self.place = placements(self.shape)
        # per-block parameters the engine reads: fused W', q/k/v bias, norms
        self.operands = [{k: torch.empty_like(v) for k, v in eng.wq.items()} for _ in range(L)]
        self.params = []
        for blk in model.blocks:
            eng.set_block(blk.weights)
            self.params.append((eng.bias_qkv, eng.norm_in, eng.norm_post))
        if keep_activations is None:
            per_block = sum(t.numel() * t.element_size() for t in eng.new_activations().values())
            free, _ = torch.cuda.mem_get_info(self.device)
            keep_activations = per_block * L < free // 2
        self.acts = [eng.new_activations() for _ in range(L)] if keep_activations else None
        self.stream = [torch.empty(T, h, dtype=f32, device=self.device) for _ in range(L + 1)]
        self.grads = [torch.empty(T, h, dtype=f32, device=self.device) for _ in range(2)]
        self.scratch = None if keep_activations else torch.empty(T, h, dtype=f32, device=self.device)
        # head
        self.vocab = V = int(head.shape[0])
        if head.shape[1] != h:
            raise ArchitectureError(f"head is {tuple(head.shape)}, hidden size {h}")
        if Vp == V and head.dtype == bf and head.is_contiguous():
            self.head = head
        else:
            self.head = torch.zeros(Vp, h, dtype=bf, device=self.device)
            self.head[:V].copy_(head)
        self.final_norm = model.norm.float().contiguous()
        self.xn = torch.empty(T, h, dtype=bf, device=self.device)
        self.rstd = torch.empty(T, dtype=f32, device=self.device)
        self.logits = torch.zeros(T, Vp, dtype=bf, device=self.device)  # pad columns stay zero
        self.dxn = torch.empty(T, h, dtype=f32, device=self.device)
        self.row_loss = torch.empty(T, dtype=f32, device=self.device)
        self.loss = torch.empty(1, dtype=f32, device=self.device)
        self.ids = torch.zeros(batch, S, dtype=torch.int32, device=self.device)
        self.labels = torch.full((batch, S), -1, dtype=torch.int32, device=self.device)

    # ------------------------------------------------------------- weights --
    def set_weights(self, schemes: Mapping[str, QuantScheme | None], *, eps: float = DEFAULT_EPS_FP32,
                    grids: Mapping[str, torch.Tensor] | None = None) -> None:
        """W' of every block linear: round to nearest under ``schemes[path]``
        (the searched scale from ``grids[path]`` where the scheme searches), or
        the dense weight rounded to bf16 where the path is absent or None."""
        grids = grids or {}
        for b, blk in enumerate(self.model.blocks):
            ops = self.operands[b]
            for name in LAYERS:
                path = f"{blk.name}.{name}"
                w = blk.weights.linears[name]
                p = self.place[name]
                scheme = schemes.get(path)
                if scheme is None:
                    place(ops[p.operand], w.to(torch.bfloat16), p)
                    continue
                grid = grids.get(path)
                if grid is not None:
                    grid = grid.view(w.shape[0], -1)
                K.fq_forward_mapped(w.contiguous(), None, None, None, bits=scheme.bits,
                                    group_size=scheme.group_size, mode=mode_of(scheme), eps=eps,
                                    wq_out=ops[p.operand], row_block=p.row_block,
                                    row_stride=p.row_stride, row_offset=p.row_offset,
                                    init_scale=grid)

    def _bind_block(self, b: int) -> None:
        eng = self.eng
        eng.wq = self.operands[b]
        eng.bias_qkv, eng.norm_in, eng.norm_post = self.params[b]

    # ---------------------------------------------------------------- pass --
    def run(self, tokens: torch.Tensor,
            on_block: Callable[[int, dict[str, torch.Tensor]], None] | None = None) -> torch.Tensor:
        """Forward and backward for one batch of token ids ``[n, seq_len]``
        (n <= batch). ``on_block(i, dw)`` receives block i's dL/dW' (fused
        layout, valid until the next block's backward) from the last block to
        the first. Returns the mean loss as a device scalar."""
        if tokens.dim() != 2 or tokens.shape[1] != self.seq_len or not 1 <= tokens.shape[0] <= self.batch:
            raise CalibrationError(f"a scoring batch is [<= {self.batch}, {self.seq_len}] token ids, "
                                   f"got {tuple(tokens.shape)}")
        n = tokens.shape[0]
        tok = tokens.to(device=self.device, dtype=torch.int32)
        self.ids[:n, :self.n_in].copy_(tok[:, :-1])
        self.ids[n:].zero_()
        self.labels.fill_(-1)
        self.labels[:n, :self.n_in].copy_(tok[:, 1:])
        eng, s, L = self.eng, self.shape, len(self.model.blocks)
        T, h = self.tokens, s.hidden
        K.embed_rows(self.model.embed, self.ids.view(-1), self.stream[0])
        keep = self.acts is not None
        for b in range(L):
            self._bind_block(b)
            if keep:
                eng.bind(self.acts[b])
            eng.forward(self.stream[b], self.stream[b + 1], save=keep)
        # head and loss
        V = self.vocab
        K.rmsnorm_fwd(self.stream[L], self.final_norm, s.norm_eps, self.xn, self.rstd)
        K.gemm("nt", self.xn, self.head, self.logits, M=T, N=self.logits.shape[1], K=h,
               workspace=eng.gemm_ws)
        K.cross_entropy(self.logits, self.labels.view(-1), V=V, scale=1.0 / (n * self.n_in),
                        row_loss=self.row_loss, loss_out=self.loss, dlogits=self.logits)
        K.gemm("nn", self.logits, self.head, self.dxn, M=T, N=h, K=self.logits.shape[1],
               workspace=eng.gemm_ws)
        cur, nxt = self.grads
        K.rmsnorm_bwd(self.dxn, self.stream[L], self.final_norm, self.rstd, None, dh_f32=cur)
        for b in reversed(range(L)):
            self._bind_block(b)
            if keep:
                eng.bind(self.acts[b], self.stream[b])
            else:
                eng.forward(self.stream[b], self.scratch, save=True)
            eng.grad_out = cur
            eng.backward(dx_out=nxt if b > 0 else None)
            if on_block is not None:
                on_block(b, eng.dw)
            cur, nxt = nxt, cur
        return self.loss
