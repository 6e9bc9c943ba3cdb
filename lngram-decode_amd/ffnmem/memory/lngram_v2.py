"""Route n-gram memory v2 on MI355X: drop-in for the reference ``ffnmem/memory/lngram_v2.py``.

Same classes, constructor signatures, attributes, ``state_dict`` keys and private
methods that the reference's callers use (``quantize_route_logits``,
``_lookup_route_chunk``, ``_project_query``, ``_project_memory``, ``_manual_gqa``,
``_real_route_probabilities``, ``_finish``; ``lngram_v2.py:1012-1131``,
``:1354-1407``, ``:1887-1920``).  Every forward op is a gfx950 kernel from
``lngram_hip``; tensors must be on a ROCm device.

Scope: the eval-mode forward, and the training-mode lookup with its surrogate route gradient
(``_LngramSurrogate``, ``lngram_v2.py:328-464``: ``_lookup_route_chunk`` with route logits under
autograd gives the route logits their counterfactual gradient and the tables their gather
gradient, both on gfx950 kernels).  The readout after the lookup has no backward here, so the
module's forward in training mode, dropout and the context-parallel / streaming-state /
packed-segment conv machinery of the reference raise ``NotImplementedError``.  The ``streaming``
execution mode computes the same function as ``full``; both run the same kernels (the fused
kernel is itself an online softmax over routes).
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import torch
from torch import Tensor, nn

from lngram_hip import ops


@torch.no_grad()
def _normal_init(weight: Tensor, std: float) -> None:
    """N(0, std) drawn in fp32, then cast (``lngram_v2.py:20-33``)."""
    if std < 0.0:
        raise ValueError(f"initialization std must be non-negative, got {std}")
    if std == 0.0:
        weight.zero_()
        return
    if weight.dtype == torch.float32:
        nn.init.normal_(weight, mean=0.0, std=std)
        return
    tmp = torch.empty_like(weight, dtype=torch.float32)
    nn.init.normal_(tmp, mean=0.0, std=std)
    weight.copy_(tmp.to(weight.dtype))


class _LngramSurrogate(torch.autograd.Function):
    """Identity on the looked-up memory of one order; the backward passes the memory gradient
    through and gives the route logits the surrogate gradient (``lngram_v2.py:328-464``),
    approximate (one-bit counterfactual rows) or exact (alphabet expectation), on
    ``lng_surrogate_grad``.  Same arguments as the reference's."""

    @staticmethod
    def forward(ctx, hard_memory: Tensor, q_logits: Tensor, route_codes: Tensor, table_weight: Tensor,
                valid_mask: Tensor, order: int, bits: int, route_start: int, alphabet_size: int,
                temperature: float, scale: float, exact: bool, hard_is_lookup: Optional[bool] = None) -> Tensor:
        """``hard_is_lookup`` (not in the reference; the lookup of this module passes True): the
        memory is the lookup's own rows, ``table[row] * valid``, so the backward reads them from the
        table instead of keeping a copy."""
        if int(alphabet_size) != 1 << int(bits):
            raise ValueError("alphabet_size must be 2**bits")
        from_table = bool(hard_is_lookup)
        saved = (q_logits, route_codes, table_weight, valid_mask)
        ctx.save_for_backward(*(saved if from_table else saved + (hard_memory.detach(),)))
        ctx.cfg = (int(order), int(bits), int(route_start), float(temperature), float(scale), bool(exact))
        ctx.n_inputs = 12 if hard_is_lookup is None else 13
        return hard_memory

    @staticmethod
    def backward(ctx, grad_memory: Optional[Tensor]):
        if grad_memory is None:
            return (None,) * ctx.n_inputs
        saved = ctx.saved_tensors
        q_logits, codes, table, valid_mask = saved[:4]
        hard = saved[4] if len(saved) > 4 else None
        order, bits, route_start, temperature, scale, exact = ctx.cfg
        grad_q = ops.surrogate_grad(grad_memory, hard, q_logits.detach(), codes, table.detach(), valid_mask, order,
                                    bits, route_start, temperature, scale, exact)
        return (grad_memory, grad_q) + (None,) * (ctx.n_inputs - 2)


class _TableRows(torch.autograd.Function):
    """One order's looked-up rows ``[B, T, R, D]`` (zero where masked; ``lng_route_tokens``) with
    the gather's table gradient (``lng_table_grad``), the embedding backward of
    ``lngram_v2.py:1084-1092``."""

    @staticmethod
    def forward(ctx, table: Tensor, route_codes: Tensor, codes_chunk: Tensor, valid_mask: Tensor, order: int,
                bits: int, route_start: int, route_end: int, segment_ids: Optional[Tensor],
                valid_tokens: Optional[Tensor]) -> Tensor:
        ctx.save_for_backward(codes_chunk, valid_mask)
        ctx.cfg = (int(order), int(bits), int(route_start), table.shape[0], table.dtype)
        return ops.route_tokens(route_codes, [table.detach()], [int(order)], int(bits), int(route_start),
                                int(route_end), segment_ids, valid_tokens, None)

    @staticmethod
    def backward(ctx, grad: Tensor):
        codes_chunk, valid_mask = ctx.saved_tensors
        order, bits, route_start, rows, dtype = ctx.cfg
        g = ops.table_grad(grad, codes_chunk, valid_mask, order, bits, route_start, rows)
        return (g.to(dtype),) + (None,) * 9


class RMSNorm(nn.Module):
    """RMSNorm (``lngram_v2.py:36-53``): ``F.rms_norm`` semantics, the row normalised and
    multiplied by ``weight`` in fp32 and rounded once to the input dtype.  Runs ``lng_rmsnorm``."""

    def __init__(self, hidden_size: int, eps: float = 1e-6, device=None, dtype=None):
        super().__init__()
        self.hidden_size = int(hidden_size)
        self.eps = float(eps)
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))

    def forward(self, hidden_states: Tensor) -> Tensor:
        if hidden_states.shape[-1] != self.hidden_size:
            raise ValueError(f"RMSNorm expects last dim {self.hidden_size}, got {hidden_states.shape[-1]}")
        return ops.rmsnorm(hidden_states, self.weight, self.eps, fused=True)


def build_lngram_norm(normalization: str, hidden_size: int, eps: float, device=None, dtype=None) -> nn.Module:
    """``lngram_v2.py:56-71``.  Only RMSNorm has a kernel; LayerNorm is rejected."""
    name = str(normalization).lower().replace("_", "")
    if name == "rmsnorm":
        return RMSNorm(hidden_size, eps=eps, device=device, dtype=dtype)
    if name == "layernorm":
        raise NotImplementedError("LNGram LayerNorm readout has no MI355X kernel; use RMSNorm")
    raise ValueError(f"Unsupported LNGram normalization {normalization!r}; expected RMSNorm or LayerNorm")


def pack_bits_to_route_codes(bits: Tensor, bits_per_route: int) -> Tensor:
    """Pack ``[B,T,R*M]`` binary channels into int32 route codes ``[B,T,R]`` (``lngram_v2.py:74-89``)."""
    if bits.dim() != 3:
        raise ValueError(f"bits must be [B,T,C], got {tuple(bits.shape)}")
    channels = bits.shape[-1]
    bits_per_route = int(bits_per_route)
    if bits_per_route <= 0 or bits_per_route > 30 or channels % bits_per_route:
        raise ValueError(f"channels={channels} must be divisible by bits_per_route in [1,30], got {bits_per_route}")
    if bits_per_route > 8:
        raise NotImplementedError("route codes wider than 8 bits have no kernel")
    return ops.pack_route_codes(bits.to(torch.float32), bits_per_route, torch.int32)


def route_code_storage_dtype(bits_per_route: int) -> torch.dtype:
    """Smallest dtype that holds every code (``lngram_v2.py:92-101``)."""
    bits_per_route = int(bits_per_route)
    if bits_per_route <= 0 or bits_per_route > 16:
        raise ValueError(f"bits_per_route must be in [1, 16], got {bits_per_route}")
    if bits_per_route <= 8:
        return torch.uint8
    if bits_per_route <= 15:
        return torch.int16
    return torch.int32


def _aligned_ngram_address(codes: Tensor, order: int, bits: int) -> Tensor:
    """Valid-window addresses ``[B, T-order+1, R]``, oldest digit first (``lngram_v2.py:314-325``)."""
    out = torch.int64 if codes.dtype == torch.int64 else torch.int32
    return ops.ngram_address(codes, order, bits, out)


class DepthwiseCausalConv(nn.Module):
    """Zero-left-padded depthwise causal conv (``lngram_v2.py:207-286``): ``SiLU(conv(RMSNorm(x)))``.

    Parameters ``norm.weight`` and ``conv.weight [d, 1, K]`` as in the reference; the
    forward runs ``lng_causal_conv``."""

    def __init__(self, hidden_size: int, kernel_size: int, dilation: int, eps: float, normalization: str = "RMSNorm",
                 bias: bool = False, zero_init: bool = True, device=None, dtype=None):
        super().__init__()
        self.hidden_size = int(hidden_size)
        self.kernel_size = int(kernel_size)
        self.dilation = int(dilation)
        self.left_padding = (self.kernel_size - 1) * self.dilation
        self.norm = build_lngram_norm(normalization, hidden_size, eps, device=device, dtype=dtype)
        self.conv = nn.Conv1d(hidden_size, hidden_size, kernel_size=self.kernel_size, dilation=self.dilation,
                              groups=hidden_size, bias=bias, device=device, dtype=dtype)
        self.act = nn.SiLU()
        if zero_init:
            nn.init.zeros_(self.conv.weight)
            if self.conv.bias is not None:
                nn.init.zeros_(self.conv.bias)

    def _check(self, values: Tensor, segment_ids) -> None:
        if values.dim() != 3 or values.shape[-1] != self.hidden_size:
            raise ValueError(f"causal conv expects [B,T,{self.hidden_size}], got {tuple(values.shape)}")
        if segment_ids is not None:
            raise NotImplementedError("packed-segment causal conv is not part of the MI355X path")
        if self.conv.bias is not None:
            raise NotImplementedError("conv bias is not supported by lng_causal_conv")

    def forward(self, values: Tensor, segment_ids: Optional[Tensor] = None) -> Tensor:
        self._check(values, segment_ids)
        return ops.causal_conv(values, self.norm.weight, self.conv.weight, self.dilation, self.norm.eps,
                               residual=False)

    def forward_incremental(self, values: Tensor, history: Optional[Tensor]) -> Tuple[Tensor, Tensor]:
        """``forward_incremental`` (``lngram_v2.py:288-311``): the output for ``values [B, n, H]``
        that follow ``history [B, H, left_padding]`` (None at the sequence start), and the history
        of the next call.  Here the history holds the last ``left_padding`` input rows before their
        RMSNorm: ``lng_causal_conv_at`` normalises every row it reads exactly as the whole-sequence
        conv does, so chained calls give the whole sequence's output bit for bit (a zero row
        normalises to zero, the left padding)."""
        self._check(values, None)
        b, n, d = values.shape
        lp = self.left_padding
        if lp == 0:
            return self.forward(values), values.new_zeros(b, d, 0)
        if history is None:
            hist_rows = values.new_zeros(b, lp, d)
        else:
            if tuple(history.shape) != (b, d, lp):
                raise ValueError(f"conv history shape={tuple(history.shape)}, expected {(b, d, lp)}")
            hist_rows = history.transpose(1, 2).to(values.dtype)
        window = torch.cat((hist_rows, values), dim=1).contiguous()
        out = ops.causal_conv_at(window, self.norm.weight, self.conv.weight, self.dilation, self.norm.eps, pos0=lp,
                                 n=n, residual=False)
        return out, window[:, -lp:].transpose(1, 2).contiguous()

    def forward_residual(self, values: Tensor) -> Tensor:
        """``values + forward(values)`` in one kernel (the ``_finish`` residual)."""
        self._check(values, None)
        return ops.causal_conv(values, self.norm.weight, self.conv.weight, self.dilation, self.norm.eps,
                               residual=True)

    def takes_row_stats(self, dtype: torch.dtype) -> bool:
        """Whether :meth:`forward_residual_stats` applies (bf16, kernel 4, dilation 3, no bias)."""
        return (dtype == torch.bfloat16 and self.kernel_size == 4 and self.dilation == 3
                and self.conv.bias is None and self.hidden_size % 8 == 0 and self.hidden_size <= 2048)

    def forward_residual_stats(self, values: Tensor, rowsq: Tensor) -> Tensor:
        """:meth:`forward_residual` with the RMSNorm row statistics computed by the producing
        projection (``ops.linear_rowsq``)."""
        self._check(values, None)
        return ops.causal_conv_rowsq(values, rowsq, self.norm.weight, self.conv.weight, self.dilation,
                                     self.norm.eps, residual=True)


class _RouteNgramMemoryBase(nn.Module):
    """Hard route n-gram tables followed by a GQA route-memory readout (``lngram_v2.py:842-1010``)."""

    def __init__(self, hidden_size: int, bits_per_route: int = 4, num_routes: int = 16, memory_dim: int = 128,
                 ngrams: Sequence[int] = (2, 3), initializer_range: float = 0.02, table_init_std_scale: float = 0.0,
                 output_proj_init_std_scale: float = 1.0, readout_q_proj_init_std_scale: float = 1.0,
                 readout_kv_proj_init_std_scale: float = 1.0, readout_num_heads: int = 16,
                 readout_num_kv_heads: int = 2, readout_head_dim: int = 128, readout_attention_dropout: float = 0.0,
                 rmsnorm_eps: float = 1e-6, normalization: str = "RMSNorm", conv_kernel_size: int = 4,
                 conv_dilation: Optional[int] = None, conv_bias: bool = False, conv_zero_init: bool = True,
                 execution_mode: str = "full", auto_max_kv_mb: float = 384.0, stream_route_chunk_size: int = 64,
                 readout_checkpoint_streaming: bool = False, q_surrogate_enable: bool = True,
                 q_surrogate_mode: str = "approximate", q_surrogate_temperature: float = 1.0,
                 q_surrogate_scale: float = 1.0, dropout: float = 0.0, device=None, dtype=None):
        super().__init__()
        self.hidden_size = int(hidden_size)
        self.bits_per_route = int(bits_per_route)
        self.num_routes = int(num_routes)
        self.memory_dim = int(memory_dim)
        if self.hidden_size <= 0:
            raise ValueError("hidden_size must be positive")
        if self.bits_per_route <= 0 or self.bits_per_route > 16:
            raise ValueError("bits_per_route must be in [1, 16]; larger code spaces make "
                             "the exact surrogate and n-gram tables impractical")
        if self.num_routes <= 0 or self.memory_dim <= 0:
            raise ValueError("num_routes and memory_dim must be positive")
        if float(table_init_std_scale) < 0.0:
            raise ValueError("table_init_std_scale must be non-negative")
        if not 0.0 <= float(dropout) < 1.0:
            raise ValueError("dropout must be in [0, 1)")
        if not 0.0 <= float(readout_attention_dropout) < 1.0:
            raise ValueError("readout_attention_dropout must be in [0, 1)")
        if float(auto_max_kv_mb) <= 0.0:
            raise ValueError("auto_max_kv_mb must be positive")
        if int(stream_route_chunk_size) <= 0:
            raise ValueError("stream_route_chunk_size must be positive")
        if float(q_surrogate_temperature) < 0.0:
            raise ValueError("q_surrogate_temperature must be non-negative")
        if int(conv_kernel_size) <= 0:
            raise ValueError("conv_kernel_size must be positive")
        if conv_dilation is not None and int(conv_dilation) <= 0:
            raise ValueError("conv_dilation must be positive when supplied")
        self.ngrams = tuple(sorted({int(v) for v in ngrams}))
        if not self.ngrams or min(self.ngrams) < 1:
            raise ValueError(f"invalid n-gram orders: {self.ngrams}")
        self.max_ngram_order = max(self.ngrams)
        self.route_history_length = self.max_ngram_order - 1
        self.route_history_dtype = route_code_storage_dtype(self.bits_per_route)
        self.alphabet_size = 1 << self.bits_per_route
        self.route_logits_dim = self.num_routes * self.bits_per_route
        self.route_token_dim = len(self.ngrams) * self.memory_dim

        self.readout_num_heads = int(readout_num_heads)
        self.readout_num_kv_heads = int(readout_num_kv_heads)
        self.readout_head_dim = int(readout_head_dim)
        if self.readout_num_heads <= 0 or self.readout_num_kv_heads <= 0 or self.readout_head_dim <= 0:
            raise ValueError("readout head counts and head dimension must be positive")
        if self.readout_num_heads % self.readout_num_kv_heads:
            raise ValueError("readout_num_heads must be divisible by readout_num_kv_heads")
        if self.readout_num_heads * self.readout_head_dim != self.hidden_size:
            raise ValueError("LNGram GQA must preserve the full query width: readout_num_heads * readout_head_dim "
                             f"must equal hidden_size; got {self.readout_num_heads} * {self.readout_head_dim} != "
                             f"{self.hidden_size}")
        self.readout_groups = self.readout_num_heads // self.readout_num_kv_heads
        self.readout_inner_dim = self.readout_num_heads * self.readout_head_dim
        self.readout_kv_inner_dim = self.readout_num_kv_heads * self.readout_head_dim
        self.softmax_scale = self.readout_head_dim ** -0.5
        self.readout_attention_dropout = float(readout_attention_dropout)
        self.execution_mode = str(execution_mode).lower()
        if self.execution_mode not in {"full", "streaming", "auto"}:
            raise ValueError("execution_mode must be full, streaming, or auto")
        self.auto_max_kv_bytes = int(float(auto_max_kv_mb) * 1024 * 1024)
        self.stream_route_chunk_size = int(stream_route_chunk_size)
        self.readout_checkpoint_streaming = bool(readout_checkpoint_streaming)
        self.q_surrogate_enable = bool(q_surrogate_enable)
        self.q_surrogate_mode = str(q_surrogate_mode).lower()
        if self.q_surrogate_mode not in {"exact", "approximate"}:
            raise ValueError("q_surrogate_mode must be exact or approximate")
        self.q_surrogate_temperature = float(q_surrogate_temperature)
        self.q_surrogate_scale = float(q_surrogate_scale)
        max_rows = max(self.num_routes * (self.alphabet_size ** n) for n in self.ngrams)
        self.index_dtype = torch.int32 if max_rows - 1 <= torch.iinfo(torch.int32).max else torch.long

        self.tables = nn.ModuleDict()
        for n in self.ngrams:
            table = nn.Embedding(self.num_routes * (self.alphabet_size ** n), self.memory_dim, device=device,
                                 dtype=dtype)
            _normal_init(table.weight, initializer_range * table_init_std_scale)
            self.tables[f"ngram_{n}"] = table
        self.lookup_dropout = nn.Dropout(float(dropout))
        self.readout_query_norm = build_lngram_norm(normalization, hidden_size, rmsnorm_eps, device, dtype)
        self.readout_memory_norm = build_lngram_norm(normalization, self.route_token_dim, rmsnorm_eps, device, dtype)
        self.readout_q_proj = nn.Linear(hidden_size, self.readout_inner_dim, bias=False, device=device, dtype=dtype)
        self.readout_kv_proj = nn.Linear(self.route_token_dim, 2 * self.readout_kv_inner_dim, bias=False,
                                         device=device, dtype=dtype)
        self.readout_o_proj = nn.Linear(self.readout_inner_dim, hidden_size, bias=False, device=device, dtype=dtype)
        _normal_init(self.readout_q_proj.weight, initializer_range * readout_q_proj_init_std_scale)
        _normal_init(self.readout_kv_proj.weight, initializer_range * readout_kv_proj_init_std_scale)
        _normal_init(self.readout_o_proj.weight, initializer_range * output_proj_init_std_scale)
        self.short_conv = DepthwiseCausalConv(hidden_size, kernel_size=conv_kernel_size,
                                              dilation=max(self.ngrams) if conv_dilation is None else int(conv_dilation),
                                              eps=rmsnorm_eps, normalization=normalization, bias=conv_bias,
                                              zero_init=conv_zero_init, device=device, dtype=dtype)
        self._fused_cache: tuple | None = None
        self._q_fold_cache: tuple | None = None

    # ------------------------------------------------------------------ codes
    def quantize_route_logits(self, q_logits: Tensor) -> Tensor:
        """int32 codes from ``q_logits > 0`` (``lngram_v2.py:1012-1017``)."""
        if q_logits.shape[-1] != self.route_logits_dim:
            raise ValueError(f"route logits dim={q_logits.shape[-1]}, expected {self.route_logits_dim}")
        if self.bits_per_route > 8:
            raise NotImplementedError("route codes wider than 8 bits have no kernel")
        return ops.pack_route_codes(q_logits, self.bits_per_route, torch.int32)

    def _use_surrogate(self, q_logits: Optional[Tensor]) -> bool:
        return bool(self.q_surrogate_enable and self.training and torch.is_grad_enabled() and q_logits is not None)

    def _check_inference(self, q_logits: Optional[Tensor] = None) -> None:
        if self._use_surrogate(q_logits):
            raise NotImplementedError("the readout has no backward kernels: in training mode only "
                                      "_lookup_route_chunk (route rows + surrogate route gradient) runs on the GPU")
        self._check_dropout()

    def _check_dropout(self) -> None:
        if self.training and (self.lookup_dropout.p > 0 or self.readout_attention_dropout > 0):
            raise NotImplementedError("dropout in training mode is not part of the MI355X path")

    def _valid_mask(self, order: int, batch: int, time: int, device, segment_ids: Optional[Tensor],
                    valid_tokens: Optional[Tensor]) -> Tensor:
        """``lngram_v2.py:1027-1045`` (bool ``[B, T]``)."""
        valid = torch.zeros(batch, time, dtype=torch.bool, device=device)
        if time < order:
            return valid
        suffix = torch.ones(batch, time - order + 1, dtype=torch.bool, device=device)
        if segment_ids is not None:
            suffix &= segment_ids[:, : time - order + 1] == segment_ids[:, order - 1:]
        if valid_tokens is not None:
            suffix &= valid_tokens[:, order - 1:]
        valid[:, order - 1:] = suffix
        return valid

    def _lookup_route_chunk(self, route_codes: Tensor, q_logits_btrm: Optional[Tensor], route_start: int,
                            route_end: int, segment_ids: Optional[Tensor], valid_tokens: Optional[Tensor],
                            target_length: Optional[int] = None) -> Tensor:
        """Route tokens ``[B, T, route_end-route_start, len(ngrams)*mem_dim]`` (``lngram_v2.py:1047-1113``):
        ``lng_route_tokens`` gathers every order's row (zero where masked) in one pass.

        In training with route logits under autograd, each order's rows come from ``_TableRows``
        (table gradient on the backward) through ``_LngramSurrogate`` (route-logit gradient), as in
        the reference (``:1093-1109``)."""
        self._check_dropout()
        if self._use_surrogate(q_logits_btrm):
            if target_length is not None:
                raise RuntimeError("cached inference cannot use surrogate gradients")
            return self._lookup_with_surrogate(route_codes, q_logits_btrm, int(route_start), int(route_end),
                                               segment_ids, valid_tokens)
        tables = [self.tables[f"ngram_{n}"].weight for n in self.ngrams]
        tl = None if target_length is None else int(target_length)
        if tl is not None and not 0 < tl <= route_codes.shape[1]:
            # the reference slices [:, -tl:]; only 0 < tl <= T maps onto the kernel's tail window
            full = ops.route_tokens(route_codes, tables, self.ngrams, self.bits_per_route, int(route_start),
                                    int(route_end), segment_ids, valid_tokens, None)
            return full[:, -tl:]
        return ops.route_tokens(route_codes, tables, self.ngrams, self.bits_per_route, int(route_start),
                                int(route_end), segment_ids, valid_tokens, tl)

    def _lookup_with_surrogate(self, route_codes: Tensor, q_logits_btrm: Tensor, route_start: int, route_end: int,
                               segment_ids: Optional[Tensor], valid_tokens: Optional[Tensor]) -> Tensor:
        b, t, _ = route_codes.shape
        codes = route_codes[:, :, route_start:route_end].contiguous()
        q_chunk = q_logits_btrm[:, :, route_start:route_end, :]
        parts = []
        for order in self.ngrams:
            valid = self._valid_mask(order, b, t, route_codes.device, segment_ids, valid_tokens)
            table = self.tables[f"ngram_{order}"].weight
            rows = _TableRows.apply(table, route_codes, codes, valid, order, self.bits_per_route, route_start,
                                    route_end, segment_ids, valid_tokens)
            parts.append(_LngramSurrogate.apply(rows, q_chunk, codes, table, valid, order, self.bits_per_route,
                                                route_start, self.alphabet_size, self.q_surrogate_temperature,
                                                self.q_surrogate_scale, self.q_surrogate_mode == "exact", True))
        return torch.cat(parts, dim=-1)

    # ------------------------------------------------------------------ projections
    def _project_query(self, hidden_states: Tensor) -> Tensor:
        """``W_q RMSNorm(h)`` -> ``[B, T, H, hd]`` (``lngram_v2.py:1115-1118``)."""
        b, t, _ = hidden_states.shape
        q = ops.linear(self.readout_query_norm(hidden_states), self.readout_q_proj.weight)
        return q.view(b, t, self.readout_num_heads, self.readout_head_dim)

    def _project_memory(self, route_tokens: Tensor) -> Tuple[Tensor, Tensor]:
        """Memory RMSNorm + KV projection -> key, value ``[B, T, KV, R, hd]`` views (``lngram_v2.py:1120-1131``)."""
        kv = ops.linear(self.readout_memory_norm(route_tokens), self.readout_kv_proj.weight)
        key, value = kv.split(self.readout_kv_inner_dim, dim=-1)
        b, t, r, _ = key.shape
        key = key.view(b, t, r, self.readout_num_kv_heads, self.readout_head_dim).permute(0, 1, 3, 2, 4)
        value = value.view(b, t, r, self.readout_num_kv_heads, self.readout_head_dim).permute(0, 1, 3, 2, 4)
        return key, value

    def _resolve_mode(self, hidden_states: Tensor) -> str:
        """``lngram_v2.py:1339-1352`` (kept for callers; both modes run the same kernels)."""
        if self.execution_mode != "auto":
            return self.execution_mode
        b, t, _ = hidden_states.shape
        es = self.readout_kv_proj.weight.element_size()
        est = b * t * self.num_routes * (self.route_token_dim + 2 * self.readout_kv_inner_dim) * es * 2
        return "full" if est <= self.auto_max_kv_bytes else "streaming"

    def _finish(self, head_output: Tensor, segment_ids: Optional[Tensor]) -> Tensor:
        """``mixed = W_o head``; ``mixed + short_conv(mixed)`` (``lngram_v2.py:1354-1359``)."""
        b, t, _, _ = head_output.shape
        if segment_ids is not None:
            raise NotImplementedError("packed-segment causal conv is not part of the MI355X path")
        flat = head_output.reshape(b, t, self.readout_inner_dim)
        if self.short_conv.takes_row_stats(flat.dtype) and self.readout_inner_dim % 32 == 0:
            # the projection kernel also writes the conv's RMSNorm row statistics
            mixed, rowsq = ops.linear_rowsq(flat, self.readout_o_proj.weight)
            return self.short_conv.forward_residual_stats(mixed, rowsq)
        # other dtypes and widths: the projection, then the single-pass conv (row statistics formed
        # inside its blocks)
        mixed = ops.linear(flat, self.readout_o_proj.weight)
        return self.short_conv.forward_residual(mixed)

    # ------------------------------------------------------------------ fused path
    def _fused_shape_ok(self, hidden_states: Tensor, tables: bool = True) -> bool:
        """Whether the fused readout serves this layer (``tables``: reading its own tables, which
        must then be on the device, not offloaded)."""
        ok = (hidden_states.dtype == torch.bfloat16 and self.ngrams == (2, 3) and self.memory_dim == 128
              and self.bits_per_route == 4 and self.num_routes <= 256
              and self.readout_num_heads == 16 and self.readout_head_dim == 64
              and self.readout_num_kv_heads == 4 and self.readout_kv_proj.weight.dtype == torch.bfloat16
              and all(t.weight.dtype == torch.bfloat16 for t in self.tables.values()))
        if ok and tables:
            ok = all(t.weight.device.type == "cuda" for t in self.tables.values())
        return ok

    def _folded_query_weight(self) -> Tensor:
        """``readout_q_proj.weight`` with ``readout_query_norm.weight`` folded into its columns
        (``ops.fold_columns``), cached per weight version: the fused path projects the raw hidden
        states with it and lets the readout kernel apply each row's RMS scale."""
        w, n = self.readout_q_proj.weight, self.readout_query_norm.weight
        key = (w.data_ptr(), w._version, n.data_ptr(), n._version, w.device)
        if self._q_fold_cache is None or self._q_fold_cache[0] != key:
            self._q_fold_cache = (key, ops.fold_columns(w.detach(), n.detach()))
        return self._q_fold_cache[1]

    def _fused_weights(self) -> Tensor:
        """The fused readout's packed KV weight (``ops.memory_readout_pack`` of
        ``readout_kv_proj.weight``), cached per weight version."""
        w = self.readout_kv_proj.weight
        key = (w.data_ptr(), w._version, w.device)
        if self._fused_cache is None or self._fused_cache[0] != key:
            self._fused_cache = (key, ops.memory_readout_pack(w.detach()))
        return self._fused_cache[1]

    def forward(self, hidden_states: Tensor, route_codes_btr: Tensor, q_logits: Optional[Tensor] = None,
                segment_ids: Optional[Tensor] = None, valid_tokens: Optional[Tensor] = None) -> Tensor:
        """``RouteNgramMemoryV2.forward`` (``lngram_v2.py:1361-1407``), eval.

        The bf16 SB/SD shape runs ``lng_memory_readout_fused`` (gather + sink readout without
        materialising keys/values); other shapes run the materialised kernels."""
        if hidden_states.dim() != 3:
            raise ValueError("hidden_states must be [B,T,H]")
        b, t, hidden = hidden_states.shape
        if hidden != self.hidden_size:
            raise ValueError(f"hidden size={hidden}, expected {self.hidden_size}")
        if tuple(route_codes_btr.shape) != (b, t, self.num_routes):
            raise ValueError("route_codes_btr has an incompatible shape")
        q_btrm = None
        if q_logits is not None:
            expected = (b, t, self.route_logits_dim)
            if tuple(q_logits.shape) != expected:
                raise ValueError(f"q_logits shape={tuple(q_logits.shape)}, expected {expected}")
            q_btrm = q_logits.reshape(b, t, self.num_routes, self.bits_per_route)
        self._check_inference(q_btrm)
        if segment_ids is None and valid_tokens is None and self._fused_shape_ok(hidden_states):
            # the query RMSNorm's weight is folded into the projection and its row scale applied in
            # the readout kernel, so the normalised hidden states are never written out
            kv_pack = self._fused_weights()
            wq = self._folded_query_weight()
            if ops.linear_rowscale_ok(hidden_states, wq):
                # large batches: the projection kernel forms each row's RMS scale from the rows it
                # streams, so the readout reads no hidden rows
                q, q_rows = ops.linear_rowscale(hidden_states, wq, self.readout_query_norm.eps), None
            else:
                q, q_rows = ops.linear(hidden_states, wq), hidden_states
            head = ops.memory_readout_fused(q, route_codes_btr, self.tables["ngram_2"].weight,
                                            self.tables["ngram_3"].weight, kv_pack, self.readout_memory_norm.weight,
                                            self.readout_memory_norm.eps, self.softmax_scale,
                                            self.readout_sink_logit, q_rows=q_rows,
                                            q_eps=self.readout_query_norm.eps)
            head_output = head.view(b, t, self.readout_num_heads, self.readout_head_dim)
        else:
            query = self._project_query(hidden_states)
            tokens = self._lookup_route_chunk(route_codes_btr, q_btrm, 0, self.num_routes, segment_ids, valid_tokens)
            key, value = self._project_memory(tokens)
            head_output = self._manual_gqa(query, key, value)
        output = self._finish(head_output, segment_ids)
        if valid_tokens is not None:
            output = output * valid_tokens.unsqueeze(-1).to(output.dtype)
        return output

    def _manual_gqa(self, query: Tensor, key: Tensor, value: Tensor) -> Tensor:  # pragma: no cover - overridden
        raise NotImplementedError


class RouteNgramMemoryV2(_RouteNgramMemoryBase):
    """Route memory whose real entries compete with one fixed zero-value sink
    (``lngram_v2.py:1858-1920``): ``sum_i e^{s_i} v_i / (e^{b0} + sum_j e^{s_j})``,
    ``b0 = log(R (1 - m) / m)``."""

    def __init__(self, *args, sink_initial_active_mass: float = 0.5, **kwargs):
        super().__init__(*args, **kwargs)
        mass = float(sink_initial_active_mass)
        if not math.isfinite(mass) or not 0.0 < mass < 1.0:
            raise ValueError("sink_initial_active_mass must be finite and in (0, 1)")
        self.sink_initial_active_mass = mass
        self.readout_sink_logit = math.log(self.num_routes * (1.0 - mass) / mass)

    def _real_route_probabilities(self, scores: Tensor) -> Tensor:
        """Real-route probabilities with the sink in the denominator (``lngram_v2.py:1887-1897``)."""
        return ops.sink_probabilities(scores, self.readout_sink_logit)

    def _manual_gqa(self, query: Tensor, key: Tensor, value: Tensor) -> Tensor:
        """Grouped sink attention over routes (``lngram_v2.py:1899-1920``): ``lng_sink_attention``."""
        if self.training and self.readout_attention_dropout:
            raise NotImplementedError("attention dropout in training mode is not part of the MI355X path")
        b, t, _, _ = query.shape
        grouped = query.view(b, t, self.readout_num_kv_heads, self.readout_groups, self.readout_head_dim)
        out = ops.sink_attention(grouped, key, value, self.softmax_scale, self.readout_sink_logit)
        return out.reshape(b, t, self.readout_num_heads, self.readout_head_dim)
