"""Shared helpers for the parity tests (inputs, tolerances, transfers)."""
from __future__ import annotations

import numpy as np

# Parity bar on bf16 outputs (stated by the task for this path).
MAX_ABS_TOL = 2e-2
MEAN_ABS_TOL = 2e-3


def err_stats(out, ref):
    """(max-abs, mean-abs) of float arrays; NaN anywhere counts as infinite error."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if out.shape != ref.shape:
        raise AssertionError(f"shape mismatch {out.shape} vs {ref.shape}")
    if out.size == 0:
        return 0.0, 0.0
    if not np.all(np.isfinite(out)) or not np.all(np.isfinite(ref)):
        return float("inf"), float("inf")
    d = np.abs(out - ref)
    return float(d.max()), float(d.mean())


def within_tol(out, ref, max_abs=MAX_ABS_TOL, mean_abs=MEAN_ABS_TOL):
    mx, mn = err_stats(out, ref)
    return mx <= max_abs and mn <= mean_abs


def assert_close(out, ref, what="", max_abs=MAX_ABS_TOL, mean_abs=MEAN_ABS_TOL):
    mx, mn = err_stats(out, ref)
    assert mx <= max_abs and mn <= mean_abs, (
        f"{what}: max-abs {mx:.3e} (tol {max_abs:.0e}), mean-abs {mn:.3e} (tol {mean_abs:.0e})")
    return mx, mn


# Parity bar on bf16 gradients (backward): the same 2e-2 / 2e-3 figures taken
# relative to max(1, |ref|), because gradients reach |g| >> 1 where a single
# bf16 ulp already exceeds 2e-2 absolute.
GRAD_REL_TOL = 2e-2
GRAD_MEAN_TOL = 2e-3


def grad_err_stats(out, ref):
    """(max of |out-ref| / max(1,|ref|), mean|out-ref| / max(1, mean|ref|)); NaN -> inf."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if out.shape != ref.shape:
        raise AssertionError(f"shape mismatch {out.shape} vs {ref.shape}")
    if out.size == 0:
        return 0.0, 0.0
    if not np.all(np.isfinite(out)) or not np.all(np.isfinite(ref)):
        return float("inf"), float("inf")
    d = np.abs(out - ref)
    return float((d / np.maximum(1.0, np.abs(ref))).max()), float(d.mean() / max(1.0, float(np.abs(ref).mean())))


def grad_within_tol(out, ref, rel=GRAD_REL_TOL, mean=GRAD_MEAN_TOL):
    r, m = grad_err_stats(out, ref)
    return r <= rel and m <= mean


def assert_grad_close(out, ref, what="", rel=GRAD_REL_TOL, mean=GRAD_MEAN_TOL):
    r, m = grad_err_stats(out, ref)
    assert r <= rel and m <= mean, (
        f"{what}: max rel-err {r:.3e} (tol {rel:.0e}), mean rel-err {m:.3e} (tol {mean:.0e})")
    return r, m


def to_torch_bf16(a_u16, device):
    """uint16 bf16 bits (numpy) -> torch bf16 tensor on `device`."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a_u16).view(np.int16))
    return t.view(torch.bfloat16).to(device)


def from_torch_bf16(t):
    """torch bf16 tensor -> numpy uint16 bits (host copy)."""
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def gpu_normal_bf16(shape, seed, sigma, device):
    """Seeded N(0, sigma^2) bf16 tensor generated on the GPU (for GB-sized configs)."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if sigma != 1.0:
        x.mul_(sigma)
    return x.to(torch.bfloat16)


def fp8_quantize(x, scale):
    """float array / scale -> OCP e4m3 codes (uint8), round to nearest even (torch's cast)."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32) / np.float32(scale))
    # the cast turns values beyond the e4m3 range (448) into NaN
    return t.clamp_(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def make_paged(k, v, lens, page_size, rng, extra_pages=3):
    """Scatter contiguous caches k/v [B, S, Hkv, D] (any dtype) into randomly
    ordered pages [num_pages, page_size, Hkv, D] (unused pages hold garbage)
    and return (k_cache, v_cache, block_table int32 [B, max_pages])."""
    B, S, Hkv, D = k.shape
    max_pages = max(1, -(-S // page_size))
    need = [-(-int(n) // page_size) for n in lens]
    num_pages = sum(need) + extra_pages
    perm = rng.permutation(num_pages)
    kc = rng.integers(0, 256, size=(num_pages, page_size, Hkv, D)).astype(k.dtype)
    vc = rng.integers(0, 256, size=(num_pages, page_size, Hkv, D)).astype(v.dtype)
    table = np.zeros((B, max_pages), dtype=np.int32)
    nxt = 0
    for b in range(B):
        for j in range(need[b]):
            pg = int(perm[nxt])
            nxt += 1
            table[b, j] = pg
            t0, t1 = j * page_size, min((j + 1) * page_size, S)
            kc[pg, : t1 - t0] = k[b, t0:t1]
            vc[pg, : t1 - t0] = v[b, t0:t1]
    return kc, vc, table


def build_sparse_indices(seed, B, Hkv, Sq, Skv, nsparse, recent=16):
    """Key index lists shaped like the reference test's
    (examples/python/Triton/test_flash_sgqa_kernel.py:30-94): row i lists its
    `recent` latest causal keys first, then distinct keys sampled without
    replacement from the older causal range, then -1 padding.  int32
    [B, Hkv, Sq, nsparse]; numpy's generator replaces torch's."""
    rng = np.random.default_rng(seed)
    idx = np.full((B, Hkv, Sq, nsparse), -1, dtype=np.int32)
    for i in range(Sq):
        upper = min(i, Skv - 1)
        n_valid = min(nsparse, upper + 1)
        n_recent = min(recent, n_valid)
        start = upper - n_recent + 1
        if n_recent > 0:
            idx[:, :, i, :n_recent] = np.arange(start, upper + 1, dtype=np.int32)
        rest = n_valid - n_recent
        if rest > 0:
            for b in range(B):
                for h in range(Hkv):
                    idx[b, h, i, n_recent:n_recent + rest] = rng.permutation(start)[:rest]
    return idx


def gpu_sparse_indices(B, Hkv, S, nsparse, seed, device, recent=16):
    """Index lists of the reference test's shape, built on the GPU for long
    sequences: row i has min(nsparse, i + 1) usable entries, its `recent`
    latest causal keys first, then keys drawn uniformly (with replacement)
    from the older causal range, then -1 padding.  int32 [B, Hkv, S, nsparse]."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    pos = torch.arange(S, device=device, dtype=torch.int64)[:, None]
    slot = torch.arange(nsparse, device=device, dtype=torch.int64)[None, :]
    n_valid = torch.clamp(pos + 1, max=nsparse)
    n_recent = torch.clamp(n_valid, max=recent)
    start = pos - n_recent + 1                      # first recent key
    rnd = (torch.rand((B, Hkv, S, nsparse), generator=g, device=device) * start.clamp(min=1)).long()
    idx = torch.where(slot < n_recent, start + slot, rnd)
    idx = torch.where(slot < n_valid, idx, torch.full_like(idx, -1))
    return idx.to(torch.int32).contiguous()
