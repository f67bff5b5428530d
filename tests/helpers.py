"""Shared comparison helpers for the parity tests."""

import torch

# Tolerance for floating outputs (attention, norm, RoPE) against the oracle:
# bf16 outputs with fp32 accumulation.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def diff_stats(out: torch.Tensor, ref: torch.Tensor):
    d = (out.detach().float().cpu() - ref.detach().float().cpu()).abs()
    return float(d.max()) if d.numel() else 0.0, float(d.mean()) if d.numel() else 0.0


def assert_close(out, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what=""):
    assert out.shape == ref.shape, f"{what}: shape {tuple(out.shape)} != {tuple(ref.shape)}"
    o = out.detach().float().cpu()
    assert torch.isfinite(o).all(), f"{what}: non-finite output"
    mx, mn = diff_stats(out, ref)
    print(f"{what}: max_abs={mx:.3e} mean_abs={mn:.3e}", flush=True)
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max_abs={mx:.3e} (<= {max_abs}) mean_abs={mn:.3e} (<= {mean_abs})"


def assert_bitexact(out, ref, what=""):
    o, r = out.detach().cpu(), ref.detach().cpu()
    assert o.shape == r.shape and o.dtype == r.dtype, f"{what}: {o.shape}/{o.dtype} vs {r.shape}/{r.dtype}"
    same = o.view(torch.int16 if o.element_size() == 2 else torch.int32) == r.view(
        torch.int16 if r.element_size() == 2 else torch.int32
    )
    bad = int((~same).sum())
    assert bad == 0, f"{what}: {bad} of {same.numel()} elements differ"


def assert_within_ulps(out, ref, ulps=1, what=""):
    """16-bit float outputs at most `ulps` units in the last place apart
    (as ordered integers), for results of the same arithmetic summed in a
    different order."""
    o, r = out.detach().cpu(), ref.detach().cpu()
    assert o.shape == r.shape and o.dtype == r.dtype and o.element_size() == 2, what

    def ordered(t):
        i = t.view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)  # sign-magnitude -> ordered (+0 and -0 meet at 0)

    d = (ordered(o) - ordered(r)).abs()
    print(f"{what}: {int((d > 0).sum())} of {d.numel()} elements differ, at most {int(d.max())} ulp", flush=True)
    assert int(d.max()) <= ulps, f"{what}: {int(d.max())} ulp apart (<= {ulps})"
