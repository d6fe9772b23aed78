"""Comparison helpers shared by the GPU parity tests (not collected)."""
import contextlib

import torch


def oracle_arith(mode: str):
    """The oracle arithmetic a Qwen3 engine mode computes: the XCD kernel takes
    attention's products exactly (``qwen3_hir.exact_products``), the other modes
    round each one as the HIR does."""
    from oracle import qwen3_hir as O
    return O.exact_products() if mode == "xcd" else contextlib.nullcontext()


def ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    """One bf16 ulp at each element's magnitude (min normal for zeros)."""
    a = x.float().abs().clamp(min=2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def report(got: torch.Tensor, want: torch.Tensor) -> dict:
    g, w = got.detach().float().cpu().reshape(-1), want.detach().float().cpu().reshape(-1)
    err = (g - w).abs()
    scale = w.abs().max().clamp(min=1e-30)
    cos = torch.nn.functional.cosine_similarity(g, w, dim=0).item() if g.numel() > 1 else 1.0
    within_ulp = (err <= ulp_bf16(w)).float().mean().item()
    return {"max_rel": (err.max() / scale).item(), "exact": (err == 0).float().mean().item(),
            "within_1ulp": within_ulp, "cos": cos, "max_abs": err.max().item()}


def assert_close_bf16(got, want, *, max_rel=2e-2, min_exact=0.0, min_cos=0.9999, name=""):
    r = report(got, want)
    msg = f"{name}: {r}"
    assert r["max_rel"] <= max_rel, msg
    assert r["exact"] >= min_exact, msg
    assert r["cos"] >= min_cos, msg
    return r
