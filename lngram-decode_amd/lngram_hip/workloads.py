"""Synthetic workloads of the route n-gram memory hot path (shapes + seeded weights/inputs).

The shapes are the reference configurations the benchmark and the parity tests run:

- ``TINY``  tiny CPU-scale layer: d 128, 8 routes, mem_dim 32, 4 query heads x 32, 2 KV heads, fp32, 4 x 128
- ``SB``    SB-shape layer-1 memory with a hidden-state router: d 1024, 184 routes, bf16, 8 x 2048
- ``SDB``   SD-B token-routed memory (182 routes, embed2 router) for decode / drafting
- ``SDC``   SD-C: 181 routes, embed2_ssm router over a 256-channel diagonal SSM, 8 x 4096

Weights follow the module initialisers (tables, router, Q/KV projections ~N(0, 0.02));
the zero-initialised output projection and conv are re-drawn as N(0, 0.02) and N(0, 0.2)
so that the output depends on the memory, all norm weights are ones.
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import torch


@dataclass(frozen=True)
class MemoryWorkload:
    name: str
    d_model: int
    routes: int
    mem_dim: int
    q_heads: int
    kv_heads: int
    head_dim: int
    batch: int
    seq: int
    dtype: torch.dtype
    router_input: str = "hidden"
    ssm_dim: int = 0
    vocab: int = 0
    norm_eps: float = 1e-5

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    def with_shape(self, batch: int, seq: int) -> "MemoryWorkload":
        return replace(self, batch=batch, seq=seq)

    def mem_cfg(self) -> dict:
        cfg = {"routes": self.routes, "mem_dim": self.mem_dim, "kv_heads": self.kv_heads, "q_heads": self.q_heads,
               "head_dim": self.head_dim, "execution_mode": "full"}
        if self.router_input != "hidden":
            cfg["router_input"] = self.router_input
        return cfg

    def algorithmic_bytes_per_token(self) -> int:
        """HBM bytes one token of the layer forward must move at minimum: h and h_norm (or the
        router features) read, one table row per (route, order) read, the output written."""
        es = torch.finfo(self.dtype).bits // 8
        rows = self.routes * 2 * self.mem_dim * es
        act = self.d_model * es
        if self.router_input == "hidden":
            return 2 * act + rows + act
        # embed2(_ssm): h + E[x_t] read (E[x_{t-1}] is the previous token's row), s_t (fp32), out
        return 2 * act + self.ssm_dim * 4 + rows + act

    def weight_bytes(self) -> int:
        es = torch.finfo(self.dtype).bits // 8
        d, inner = self.d_model, self.q_heads * self.head_dim
        dt = 2 * self.mem_dim
        fin = {"hidden": d, "embed2": 2 * d, "embed2_ssm": 2 * d + self.ssm_dim}[self.router_input]
        router = self.routes * 4 * fin
        proj = inner * d + 2 * self.kv_heads * self.head_dim * dt + d * inner
        return (router + proj + 4 * d + dt + 2 * d) * es


TINY = MemoryWorkload("tiny d128 R8 fp32 4x128", 128, 8, 32, 4, 2, 32, 4, 128, torch.float32)
SB = MemoryWorkload("sb d1024 R184 bf16 8x2048", 1024, 184, 128, 16, 4, 64, 8, 2048, torch.bfloat16)
SDB = MemoryWorkload("sdb d1024 R182 bf16 decode", 1024, 182, 128, 16, 4, 64, 1, 2048, torch.bfloat16,
                     router_input="embed2", vocab=32768)
SDC = MemoryWorkload("sdc d1024 R181 N256 bf16 8x4096", 1024, 181, 128, 16, 4, 64, 8, 4096, torch.bfloat16,
                     router_input="embed2_ssm", ssm_dim=256, vocab=32768)


def build_memory(w: MemoryWorkload, seed: int = 0, device: str | torch.device = "cpu"):
    """``LngramMemory`` of workload ``w`` with synthetic weights, eval mode, in ``w.dtype`` on ``device``."""
    from ffnmem.memory.wrapper import LngramMemory

    torch.manual_seed(seed)
    mem = LngramMemory(w.d_model, w.mem_cfg(), init_std=0.02, norm_eps=w.norm_eps, ssm_dim=w.ssm_dim)
    g = torch.Generator().manual_seed(seed + 1)
    m = mem.module
    with torch.no_grad():
        m.readout_o_proj.weight.copy_(torch.randn(m.readout_o_proj.weight.shape, generator=g) * 0.02)
        m.short_conv.conv.weight.copy_(torch.randn(m.short_conv.conv.weight.shape, generator=g) * 0.2)
    return mem.to(w.dtype).to(device).eval()


def make_hidden(w: MemoryWorkload, seed: int = 1, device: str | torch.device = "cpu") -> torch.Tensor:
    """Hidden states ``h ~ N(0, 1)`` ``[B, T, d]`` in ``w.dtype``."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn(w.batch, w.seq, w.d_model, generator=g).to(w.dtype).to(device)


def make_tokens(w: MemoryWorkload, seed: int = 2, device: str | torch.device = "cpu") -> torch.Tensor:
    """Token ids uniform over the vocabulary ``[B, T]``."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, w.vocab, (w.batch, w.seq), generator=g).to(device)


# ----------------------------------------------------------------------------- drafter (decode) workloads
@dataclass(frozen=True)
class DraftWorkload:
    """Shape of a token-routed drafter (bundle ``config`` of ``drafting/export_drafter.py``)."""

    name: str
    d_model: int
    vocab: int
    routes: int
    mem_dim: int
    kv_heads: int
    head_dim: int
    q_heads: int
    ssm_dim: int = 0
    context: int = 2048
    dtype: torch.dtype = torch.bfloat16
    eps: float = 1e-5

    def config(self) -> dict:
        import math

        ssm = self.ssm_dim > 0
        return {"kind": "sd_c" if ssm else "sd_b", "router_kind": "embed2_ssm" if ssm else "embed2",
                "d_model": self.d_model, "vocab": self.vocab, "routes": self.routes, "bits": 4, "ngrams": [2, 3],
                "mem_dim": self.mem_dim, "kv_heads": self.kv_heads, "head_dim": self.head_dim,
                "q_heads": self.q_heads, "groups": self.q_heads // self.kv_heads,
                "route_token_dim": 2 * self.mem_dim, "ssm_dim": self.ssm_dim, "query_ssm": ssm,
                "norm_eps": self.eps, "ssm_eps": self.eps, "router_eps": self.eps, "draft_eps": self.eps,
                "mem_eps": self.eps, "softmax_scale": self.head_dim ** -0.5, "sink_logit": math.log(self.routes),
                "sketch_k": 0, "shortlist_cap": 0, "table_dtype": "bf16" if self.dtype == torch.bfloat16 else "fp32",
                "layer": 0}

    def table_params(self) -> int:
        return self.routes * (16 ** 2 + 16 ** 3) * self.mem_dim


SDB_DRAFT = DraftWorkload("sdb drafter d1024 V32768 R182 bf16", 1024, 32768, 182, 128, 4, 64, 4)
SDC_DRAFT = DraftWorkload("sdc drafter d1024 V32768 R181 N256 bf16", 1024, 32768, 181, 128, 4, 64, 4, ssm_dim=256)
TINY_DRAFT = DraftWorkload("tiny drafter d64 V512 R6", 64, 512, 6, 16, 2, 16, 4, context=96)
TINY_DRAFT_FAST = DraftWorkload("tiny drafter d64 V1000 R7 mem_dim 32", 64, 1000, 7, 32, 2, 16, 4, context=96)
TINY_DRAFT_SSM = DraftWorkload("tiny drafter d64 V512 R5 N8", 64, 512, 5, 16, 2, 16, 4, ssm_dim=8, context=96)


def build_draft_bundle(w: DraftWorkload, seed: int = 0) -> tuple[dict, dict]:
    """(config, tensors) of a synthetic drafter on the CPU: every weight ~N(0, 0.02) drawn in fp32
    and stored in ``w.dtype`` (the SSM decay ~U[0.9, 0.999] stays fp32), norm weights ones."""
    g = torch.Generator().manual_seed(seed)
    d, r, n = w.d_model, w.routes, w.ssm_dim
    kh, inner, dt = w.kv_heads * w.head_dim, w.q_heads * w.head_dim, 2 * w.mem_dim
    feat = 2 * d + (n if n else 0)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g) * 0.02).to(w.dtype)

    def ones(k):
        return torch.ones(k, dtype=w.dtype)

    t = {"embedding": rnd(w.vocab, d), "table_2": rnd(r * 16 ** 2, w.mem_dim), "table_3": rnd(r * 16 ** 3, w.mem_dim),
         "mem_norm": ones(dt), "kv_proj": rnd(2 * kh, dt), "router": rnd(r * 4, feat),
         "router_prev_norm": ones(d), "router_cur_norm": ones(d), "router_start": rnd(d),
         "q_norm": ones(d), "w_q": rnd(inner, d), "w_o": rnd(d, inner), "out_norm": ones(d)}
    if n:
        t["ssm_norm"] = ones(d)
        t["ssm_w_in"] = rnd(n, d)
        t["ssm_decay"] = 0.9 + 0.099 * torch.rand(n, generator=g)
        t["w_sq"] = rnd(inner, n)
    return w.config(), t


def make_context(w: DraftWorkload, seed: int = 0) -> list:
    """Context token ids ~U[0, vocab) (batch 1)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, w.vocab, (w.context,), generator=g).tolist()
