"""Adapter around the route memory module: drop-in for the reference ``ffnmem/memory/wrapper.py``.

Owns the router (``d_in -> R * bits``), keeps the routing logits in fp32, applies the
Lngram v2 Appendix E initialisation and exposes diagnostics (``wrapper.py:1-125``,
``:174-254``).  The router and its sign packing run as one kernel
(``lng_router_codes``: MFMA for bf16 operands, fp32 FMA otherwise); the module
forward is the fused gather + readout.  The rank-1 path (Wave 2) is not ported.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

from lngram_hip import ops

from .lngram_v2 import RouteNgramMemoryV2, _aligned_ngram_address  # noqa: F401
from .router import TokenRouter, TokenRouterFeatures, router_input_dim

# Wrapper-level keys (never passed to the module).
WRAPPER_KEYS = ("routes", "mem_dim", "kv_heads", "q_heads", "head_dim", "router_init_std", "rank1",
                "router_input", "token_router")

# Appendix E recipe (Lngram v2), overriding the module's code defaults.
APPENDIX_E = dict(
    bits_per_route=4,
    ngrams=(2, 3),
    table_init_std_scale=1.0,
    output_proj_init_std_scale=0.0,
    conv_zero_init=True,
    conv_kernel_size=4,
    q_surrogate_enable=True,
    q_surrogate_mode="approximate",
    sink_initial_active_mass=0.5,
)


class LngramMemory(nn.Module):
    """``LngramMemory(d_model, mem_cfg, init_std, norm_eps, ssm_dim)`` (``wrapper.py:50-95``)."""

    def __init__(self, d_model: int, mem_cfg: dict, init_std: float = 0.02, norm_eps: float = 1e-5,
                 ssm_dim: int = 0):
        super().__init__()
        cfg = dict(APPENDIX_E)
        cfg.update({k: v for k, v in mem_cfg.items() if k not in WRAPPER_KEYS})
        self.routes = int(mem_cfg["routes"])
        self.bits = int(cfg["bits_per_route"])
        head_dim = int(mem_cfg.get("head_dim", 64))
        q_heads = int(mem_cfg.get("q_heads", d_model // head_dim))
        if "ngrams" in cfg:
            cfg["ngrams"] = tuple(int(n) for n in cfg["ngrams"])
        self.module = RouteNgramMemoryV2(
            hidden_size=d_model,
            num_routes=self.routes,
            memory_dim=int(mem_cfg["mem_dim"]),
            readout_num_heads=q_heads,
            readout_num_kv_heads=int(mem_cfg.get("kv_heads", 4)),
            readout_head_dim=head_dim,
            initializer_range=init_std,
            rmsnorm_eps=norm_eps,
            **cfg,
        )
        self.router_input = str(mem_cfg.get("router_input", "hidden"))
        in_dim = router_input_dim(self.router_input, d_model, ssm_dim)
        self.router = nn.Linear(in_dim, self.routes * self.bits, bias=False)
        nn.init.normal_(self.router.weight, mean=0.0, std=float(mem_cfg.get("router_init_std", init_std)))
        if self.router_input != "hidden":
            self.router_features = TokenRouterFeatures(d_model, self.router_input, norm_eps, init_std)
        tr = mem_cfg.get("token_router") or {}
        self.cfg_token_router = dict(tr)
        self.token_router = None
        if tr.get("enabled", False):
            if self.router_input != "hidden":
                raise ValueError("token_router (SD-A) imitates a hidden-state router; use router_input: hidden")
            self.token_router = TokenRouter(d_model, self.routes * self.bits, norm_eps, init_std)
        self.last_route_logits: Tensor | None = None
        self.capture_route_logits = False
        self.rank1_dim = 0
        if mem_cfg.get("rank1"):
            raise NotImplementedError("the Wave 2 rank-1 memory path is not part of the MI355X build")
        self.collect_diagnostics = False
        self.reset_diagnostics()

    # ------------------------------------------------------------------ forward
    def route_logits(self, h_norm: Tensor) -> Tensor:
        """Router logits in fp32 (``wrapper.py:98-101``)."""
        logits, _ = ops.router_codes(h_norm, self.router.weight, self.bits, want_logits=True)
        return logits

    def route_codes(self, x: Tensor, want_logits: bool = False):
        """``(fp32 logits or None, uint8 codes [.., R])`` from one router + sign-pack kernel."""
        return ops.router_codes(x, self.router.weight, self.bits, want_logits=want_logits,
                                codes_dtype=torch.uint8)

    def forward(self, h: Tensor, h_norm: Tensor, router_in: Tensor | None = None) -> Tensor:
        """``wrapper.py:103-125`` (eval)."""
        if self.router_input == "hidden":
            x = h_norm
        else:
            if router_in is None:
                raise ValueError(f"router_input={self.router_input} needs router_in from the model")
            x = router_in
        keep = self.token_router is not None or self.capture_route_logits
        if self.training and torch.is_grad_enabled():
            raise NotImplementedError("training (surrogate route gradient) is not part of the MI355X path")
        q_logits, codes = self.route_codes(x, want_logits=keep)
        return self._forward_codes(h, q_logits, codes, keep)

    def forward_ids(self, h: Tensor, token_ids: Tensor, emb_table: Tensor, ssm_state: Tensor | None = None) -> Tensor:
        """``forward(h, None, router_features.from_ids(token_ids, emb_table, ssm_state))`` for a
        token-routed memory (``router.py:50-59`` + ``wrapper.py:103-125``), with the router's
        feature rows gathered inside the router GEMM from tables of the normalised embedding rows
        (``lng_router_codes_ids``), so the ``[B, T, 2d + N]`` features are never materialised.
        ``ssm_state`` ``[B, T, N]`` (``embed2_ssm``), bf16 (``ops.ssm_scan(..., want_bf16=True)``)
        or fp32.  Shapes the gathered GEMM does not take run the materialised features."""
        if self.router_input == "hidden":
            raise ValueError("forward_ids is for token-routed memories (router_input embed2 / embed2_ssm)")
        if self.training and torch.is_grad_enabled():
            raise NotImplementedError("training (surrogate route gradient) is not part of the MI355X path")
        s_in = ssm_state if self.router_input == "embed2_ssm" else None
        if self.router_input == "embed2_ssm" and s_in is None:
            raise ValueError("embed2_ssm router needs the SSM state")
        b, t = token_ids.shape
        n = 0 if s_in is None else s_in.shape[-1]
        w = self.router.weight
        if not (emb_table.dtype == w.dtype == torch.bfloat16 and self.bits == 4
                and ops.router_codes_ids_ok(b * t, emb_table.shape[1], n, w.shape[0])):
            return self.forward(h, None, self.router_features.from_ids(token_ids, emb_table, s_in))
        keep = self.token_router is not None or self.capture_route_logits
        fprev, fcur = self.router_features.tables(emb_table)
        sb = None if s_in is None else (s_in if s_in.dtype == torch.bfloat16 else s_in.to(torch.bfloat16))
        q_logits, codes = ops.router_codes_ids(token_ids, fprev, fcur, sb, w, want_logits=keep)
        return self._forward_codes(h, q_logits, codes, keep)

    def _forward_codes(self, h: Tensor, q_logits: Tensor | None, codes: Tensor, keep: bool) -> Tensor:
        if keep:
            self.last_route_logits = q_logits.detach()
        if self.collect_diagnostics and not self.training:
            self._accumulate_diagnostics(h, codes)
        return self.module(h, codes)

    # -------------------------------------------------------------- diagnostics
    def reset_diagnostics(self) -> None:
        self._code_hist = None
        self._sink_sum = 0.0
        self._sink_count = 0
        self._r1_ratio_sum = 0.0
        self._v2_ratio_sum = 0.0
        self._r1_count = 0

    @torch.no_grad()
    def _accumulate_diagnostics(self, h: Tensor, codes: Tensor) -> None:
        """Code histogram and sink mass (``wrapper.py:174-200``)."""
        m = self.module
        n_codes = 1 << self.bits
        flat = codes.reshape(-1, self.routes).long()
        counts = torch.zeros(self.routes, n_codes, device=codes.device, dtype=torch.float64)
        counts.scatter_add_(1, flat.t(), torch.ones_like(flat.t(), dtype=torch.float64))
        self._code_hist = counts if self._code_hist is None else self._code_hist + counts
        query = m._project_query(h)
        tokens = m._lookup_route_chunk(codes, None, 0, m.num_routes, None, None)
        key, _ = m._project_memory(tokens)
        b, t = query.shape[:2]
        grouped = query.view(b, t, m.readout_num_kv_heads, m.readout_groups, m.readout_head_dim)
        scores = torch.matmul(grouped.float(), key.transpose(-1, -2).float().contiguous()) * m.softmax_scale
        real = m._real_route_probabilities(scores)
        sink = 1.0 - real.sum(-1)
        self._sink_sum += float(sink.sum())
        self._sink_count += sink.numel()

    def diagnostics(self) -> dict:
        """``wrapper.py:202-220``."""
        out: dict = {}
        if self._sink_count:
            out["sink_mass"] = self._sink_sum / self._sink_count
        if self._code_hist is not None:
            p = self._code_hist / self._code_hist.sum(-1, keepdim=True).clamp_min(1)
            entropy = -(p * p.clamp_min(1e-30).log()).sum(-1)
            eff = entropy.exp()
            out["eff_codes_mean"] = float(eff.mean())
            out["frac_routes_eff_lt4"] = float((eff < 4).double().mean())
            out["frac_routes_eff_lt2"] = float((eff < 2).double().mean())
            out["dead_code_frac"] = float((self._code_hist == 0).double().mean())
            out["top_code_share"] = float(p.max(-1).values.mean())
        return out

    # ------------------------------------------------------------ bookkeeping
    @property
    def sink_initial_mass(self) -> float:
        return 1.0 - self.module.sink_initial_active_mass

    def table_parameters(self):
        return list(self.module.tables.parameters())

    def active_table_params_per_token(self) -> int:
        return self.routes * len(self.module.ngrams) * self.module.memory_dim

