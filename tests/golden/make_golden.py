"""Write the golden fixtures of ``tests/golden/*.npz`` from the reference's own modules.

    python tests/golden/make_golden.py --ref /root/reference

Run only where the reference checkout is present (it never travels with this repository).
Inputs and parameters come from ``recipe.py``; each fixture stores what the reference computed
from them, plus the torch version that computed it.  Fixtures:

- ``router_features.npz``: ``TokenRouterFeatures.forward`` / ``.step`` (``router.py:50-68``),
  embed2 and embed2_ssm, fp32 and bf16 embeddings;
- ``ssm.npz``: ``DiagonalSSM.inputs`` / ``.forward`` / ``.step`` and ``sequential_scan``
  (``ssm.py:37-65``) at a length that is not a multiple of the chunk;
- ``memory_tiny_fp32.npz``: ``LngramMemory.forward`` (``wrapper.py:103-125``) at the C1 widths;
- ``memory_sb_bf16.npz``: the same module cast to bf16 at the SB widths (32 routes), so the
  reference's bf16 rounding sequence (``lngram_v2.py:1361-1407``) is recorded;
- ``surrogate.npz``: the route-logit and memory gradients of ``_LngramSurrogate``
  (``lngram_v2.py:328-464``), approximate and exact, for the cases of ``recipe.SURROGATE_CASES``;
- ``online_counts.npz``: ``OnlineCounts(codes, x, orders, 4, V, kappa).mix(p, win, real, deadline)``
  (``drafters.py:117-142``) for the cases of ``recipe.ONLINE_CASES``;
- ``drafter_<kind>[_sketch].npz``: ``RefDrafter.trace`` (full vocabulary and shortlist) and
  ``RefDrafter.draft`` after a commit, with and without hypothetical tokens
  (``cpu_drafter.py:247-289``) on tiny SD-B / SD-C bundles, with and without count sketches.
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import recipe  # noqa: E402


def _bits(x: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> its uint16 bit patterns."""
    return x.contiguous().view(torch.int16).numpy().view(np.uint16)


def _load(module: torch.nn.Module, base: int) -> dict:
    shapes = {k: tuple(v.shape) for k, v in module.state_dict().items()}
    params = recipe.state(shapes, base)
    module.load_state_dict({k: torch.from_numpy(v) for k, v in params.items()}, strict=True)
    return shapes


def router_features(out: Path) -> None:
    from ffnmem.memory.router import TokenRouterFeatures

    d, n, b, t = 64, 16, 2, 6
    res = {"torch": np.array(torch.__version__)}
    for kind in ("embed2", "embed2_ssm"):
        f = TokenRouterFeatures(d, kind, eps=1e-5)
        _load(f, 11)
        for dt_name, dt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
            f = f.to(dt) if dt_name == "bf16" else f
            emb = torch.from_numpy(recipe.normal("rf_emb", (b, t, d))).to(dt)
            s = torch.from_numpy(recipe.normal("rf_ssm", (b, t, n))) if kind == "embed2_ssm" else None
            with torch.no_grad():
                y = f(emb, s)
                s0 = f.step(None, emb[:, 0], None if s is None else s[:, 0])
                s3 = f.step(emb[:, 2], emb[:, 3], None if s is None else s[:, 3])
            key = f"{kind}_{dt_name}"
            conv = _bits if dt_name == "bf16" else (lambda x: x.numpy())
            res[f"{key}_out"] = conv(y)
            res[f"{key}_step0"] = conv(s0)
            res[f"{key}_step3"] = conv(s3)
            f = f.float()
    np.savez_compressed(out / "router_features.npz", **res)


def ssm(out: Path) -> None:
    from ffnmem.memory.ssm import DiagonalSSM, chunked_scan, sequential_scan

    d, n, b, t = 48, 16, 2, 21
    m = DiagonalSSM(d, n, chunk=8, eps=1e-5)
    theta = m.theta.detach().clone()           # the reference's geometric init of theta
    _load(m, 12)
    with torch.no_grad():
        m.theta.copy_(theta)
        emb = torch.from_numpy(recipe.normal("ssm_emb", (b, t, d)))
        u = m.inputs(emb)
        s = m.forward(emb)
        seq = sequential_scan(m.decay(), u)
        ch4 = chunked_scan(m.decay(), u, 4)
        st = None
        steps = []
        for i in range(3):
            st = m.step(st, emb[:, i])
            steps.append(st)
    np.savez_compressed(out / "ssm.npz", torch=np.array(torch.__version__), theta=theta.numpy(), u=u.numpy(),
                        s=s.numpy(), sequential=seq.numpy(), chunked4=ch4.numpy(),
                        steps=torch.stack(steps, 1).numpy())


def _memory(spec: dict, base: int, b: int, t: int, dtype, name: str, out: Path) -> None:
    from ffnmem.memory.wrapper import LngramMemory
    from ffnmem.model import RMSNorm

    mem = LngramMemory(spec["d_model"], dict(spec["cfg"])).eval()
    _load(mem, base)
    mem = mem.to(dtype)
    d = spec["d_model"]
    h = torch.from_numpy(recipe.normal(f"{name}_h", (b, t, d))).to(dtype)
    norm = RMSNorm(d, 1e-5).to(dtype)
    with torch.no_grad():
        h_norm = norm(h)
        q = mem.route_logits(h_norm)
        codes = mem.module.quantize_route_logits(q)
        y = mem(h, h_norm)
    conv = _bits if dtype == torch.bfloat16 else (lambda x: x.numpy())
    np.savez_compressed(out / f"{name}.npz", torch=np.array(torch.__version__), h_norm=conv(h_norm),
                        q_logits=q.float().numpy(), codes=codes.numpy().astype(np.int32), out=conv(y))


def memory(out: Path) -> None:
    _memory(recipe.TINY_MEM, 21, 2, 16, torch.float32, "memory_tiny_fp32", out)
    _memory(recipe.SB_MEM, 22, 1, 24, torch.bfloat16, "memory_sb_bf16", out)


def drafter(out: Path) -> None:
    from drafting.cpu_drafter import RefDrafter
    from drafting.export_drafter import Bundle

    for kind in ("sdb", "sdc"):
        for sk in (0, 4):
            cfg = recipe.drafter_config(kind, sketch_k=sk, cap=6)
            arrays = recipe.drafter_arrays(cfg, 31)
            d = RefDrafter(Bundle(cfg, arrays, {}), topk=3)
            toks = recipe.integers(f"{kind}_tokens", (40,), 0, cfg["vocab"])
            res = {"torch": np.array(torch.__version__), "tokens": toks}
            c, ids, lg = d.trace(toks, full=True)
            res.update(full_codes=c, full_logits=lg)
            if sk:
                c2, ids2, lg2 = d.trace(toks, full=False)
                assert (c2 == c).all()
                res.update(sl_ids=ids2, sl_logits=lg2)
            d.commit(toks[:20])
            o = d.draft(4)
            res.update(draft_tokens=np.array(o.tokens), draft_ids=o.topk_ids, draft_logits=o.topk_logits,
                       draft_codes=o.codes)
            o = d.draft(3, hyp=[int(toks[25]), int(toks[26])], last_codes=True)
            res.update(hyp_tokens=np.array(o.tokens), hyp_ids=o.topk_ids, hyp_logits=o.topk_logits,
                       hyp_codes=o.codes)
            name = f"drafter_{kind}" + ("_sketch" if sk else "")
            np.savez_compressed(out / f"{name}.npz", **res)


def surrogate(out: Path) -> None:
    from ffnmem.memory.lngram_v2 import _LngramSurrogate, _aligned_ngram_address

    res = {"torch": np.array(torch.__version__)}
    for case in recipe.SURROGATE_CASES:
        name, order, bits, R, rs, B, T, D, dt_name, temp, scale, exact = case
        dt = torch.bfloat16 if dt_name == "bf16" else torch.float32
        x = recipe.surrogate_inputs(case)
        table = torch.from_numpy(x["table"]).to(dt)
        codes = torch.from_numpy(x["codes"])
        valid = torch.zeros(B, T, dtype=torch.bool)               # _valid_mask with valid_tokens
        valid[:, order - 1:] = torch.from_numpy(x["valid_tokens"])[:, order - 1:]
        A = 1 << bits
        addr = _aligned_ngram_address(codes, order, bits)
        rows = (torch.arange(rs, rs + R) * A ** order).view(1, 1, R) + addr
        hard = torch.cat((table.new_zeros(B, order - 1, R, D), table[rows]), 1) * valid[..., None, None].to(dt)
        q = torch.from_numpy(x["q"]).requires_grad_()
        mem = hard.clone().requires_grad_()
        y = _LngramSurrogate.apply(mem, q, codes, table, valid, order, bits, rs, A, temp, scale, exact)
        y.backward(torch.from_numpy(x["grad"]).to(dt))
        res[f"{name}_grad_q"] = q.grad.numpy()
        res[f"{name}_grad_mem"] = (_bits if dt == torch.bfloat16 else (lambda v: v.numpy()))(mem.grad)
    np.savez_compressed(out / "surrogate.npz", **res)


def online(out: Path) -> None:
    from drafting.drafters import OnlineCounts

    res = {"torch": np.array(torch.__version__)}
    for case in recipe.ONLINE_CASES:
        name, T, R, V, orders, kappa = case
        x = recipe.online_inputs(case)
        oc = OnlineCounts(torch.from_numpy(x["codes"]), torch.from_numpy(x["x"]), orders, 4, V, kappa)
        with torch.no_grad():
            mixed = oc.mix(torch.from_numpy(x["p"]), torch.from_numpy(x["win"]), torch.from_numpy(x["real"]),
                           torch.from_numpy(x["deadline"]))
        res[f"{name}_mix"] = mixed.numpy()
    np.savez_compressed(out / "online_counts.npz", **res)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", required=True, help="the reference checkout")
    ap.add_argument("--out", default=str(HERE))
    ap.add_argument("--only", nargs="*", help="fixture groups to write (default: all)")
    args = ap.parse_args()
    sys.path.insert(0, str(Path(args.ref).resolve()))
    torch.manual_seed(0)
    out = Path(args.out)
    groups = {"router_features": router_features, "ssm": ssm, "memory": memory, "drafter": drafter,
              "surrogate": surrogate, "online": online}
    for name in args.only or groups:
        groups[name](out)
    for p in sorted(out.glob("*.npz")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
