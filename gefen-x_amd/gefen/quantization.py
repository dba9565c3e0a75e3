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


def save_distribution_histogram_pt_from_counts(hist, prefix, suffix, num_samples, value_range=(-1.0, 1.0)):
    if prefix is None:
        raise ValueError("Cannot save gradient histogram because SAVE_CODEBOOK_PREFIX is None.")
    if hist.dim() != 1:
        raise ValueError("Expected 1D histogram counts, got dim={}.".format(hist.dim()))
    if hist.numel() <= 0:
        raise ValueError("Expected at least one histogram bin.")
    if num_samples < 0:
        raise ValueError("num_samples must be non-negative, got {}.".format(num_samples))
    prefix_path = Path(prefix).expanduser().resolve()
    prefix_path.parent.mkdir(parents=True, exist_ok=True)
    path = prefix_path.parent / "{}_{}.pt".format(prefix_path.stem, suffix)
    hist_cpu = hist.detach().cpu().to(torch.float32)
    left, right = value_range
    edges = torch.linspace(float(left), float(right), steps=hist_cpu.numel() + 1, dtype=torch.float32)
    torch.save({"hist": hist_cpu, "bin_edges": edges, "bin_centers": 0.5 * (edges[:-1] + edges[1:]),
                "bin_width": float(right - left) / float(hist_cpu.numel()),
                "range": (float(left), float(right)), "num_bins": hist_cpu.numel(),
                "num_samples": int(num_samples)}, path)
    logger.info("Saved distribution histogram data to %s", path)


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
