"""Exact-DP codebook solver (reference quantization.py).

exact_dp keeps the reference's signature and result: the optimal 256-centre
1-D weighted k-means over the active histogram bins with forced +-1 endpoints
(quantization.py:197-253), padded when there are fewer active bins than
centres (quantization.py:59-72).  The O(k n^2) float64 DP runs in the C ABI
instead of numba or pure Python: on the HIP device when one is given
(gefenx_exact_dp_device), else on host threads (gefenx_exact_dp); both make
the same float64 operations and the same first-minimum choices.
"""
from __future__ import annotations

import logging
from pathlib import Path

import numpy as np
import torch

logger = logging.getLogger(__name__)

# Optional histogram dumps (reference quantization.py module attributes).
LIST_STEPS_SAVE_HIST_GRAD = None
SAVE_CODEBOOK_PREFIX = None


def _histogram_record(counts: torch.Tensor, num_samples: int, value_range) -> dict:
    """The dumped dict (the reference's file layout: hist, bin_edges,
    bin_centers, bin_width, range, num_bins, num_samples)."""
    lo, hi = (float(v) for v in value_range)
    hist = counts.detach().to(device="cpu", dtype=torch.float32)
    nbins = hist.numel()
    edges = torch.linspace(lo, hi, steps=nbins + 1, dtype=torch.float32)
    return {"hist": hist, "bin_edges": edges, "bin_centers": (edges[1:] + edges[:-1]) * 0.5,
            "bin_width": (hi - lo) / nbins, "range": (lo, hi), "num_bins": nbins,
            "num_samples": int(num_samples)}


def save_distribution_histogram_pt_from_counts(hist, prefix, suffix, num_samples, value_range=(-1.0, 1.0)):
    """Write a histogram of normalised gradients to `<dir of prefix>/<stem of
    prefix>_<suffix>.pt` (reference quantization.py:12-56; ValueError for a
    missing prefix, non-1D or empty counts, a negative sample count)."""
    problems = [(prefix is None, "no SAVE_CODEBOOK_PREFIX is set"),
                (prefix is not None and hist.dim() != 1, "the counts must be 1D, got dim={}".format(hist.dim())),
                (prefix is not None and hist.numel() == 0, "the counts hold no bins"),
                (num_samples < 0, "num_samples must be >= 0, got {}".format(num_samples))]
    for failed, why in problems:
        if failed:
            raise ValueError("Cannot save the gradient histogram: " + why)
    target = Path(prefix).expanduser().resolve()
    out = target.with_name("{}_{}.pt".format(target.stem, suffix))
    out.parent.mkdir(parents=True, exist_ok=True)
    torch.save(_histogram_record(hist, num_samples, value_range), out)
    logger.info("Saved distribution histogram data to %s", out)


def exact_dp(histogram_stats: dict, num_codebooks: int, force_endpoints: bool = True,
             device: torch.device = None) -> torch.Tensor:
    """quantization.py:197-253.  With a HIP `device` the DP levels run there
    (gefenx_exact_dp_device, bit-identical); otherwise on host threads."""
    from gefen.kernels import _native
    centers = histogram_stats["active_centers"].detach().cpu().to(torch.float32).contiguous()
    counts = histogram_stats["active_counts"].detach().cpu().to(torch.float32).contiguous()
    if centers.numel() == 0:
        raise ValueError("Cannot run exact DP on an empty histogram.")
    if not torch.all(counts > 0):
        raise ValueError("exact DP expects strictly positive counts for all active histogram bins.")
    out = torch.empty(num_codebooks, dtype=torch.float32)
    lib = _native.load()
    if device is not None and torch.device(device).type == "cuda":
        dev = torch.device(device)
        with torch.cuda.device(dev):
            _native.check(lib.gefenx_exact_dp_device(
                centers.data_ptr(), counts.data_ptr(), centers.numel(), int(num_codebooks),
                1 if force_endpoints else 0, out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream),
                "exact_dp")
        return out
    _native.check(lib.gefenx_exact_dp(
        centers.data_ptr(), counts.data_ptr(), centers.numel(), int(num_codebooks),
        1 if force_endpoints else 0, out.data_ptr()), "exact_dp")
    return out
