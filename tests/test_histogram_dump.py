"""quantization.save_distribution_histogram_pt_from_counts (reference
quantization.py:12-56): the file name, the dict layout (hist, bin_edges,
bin_centers, bin_width, range, num_bins, num_samples) and the refusals.
The optimizer hook that calls it is tested on the GPU
(tests/test_gpu_boundary.py)."""
import os

import pytest
import torch

from gefen import quantization


def test_dump_layout(tmp_path):
    counts = torch.tensor([3, 0, 5, 2], dtype=torch.int64)
    quantization.save_distribution_histogram_pt_from_counts(counts, str(tmp_path / "run" / "cb"), "grad_hist_step_7",
                                                            10)
    path = tmp_path / "run" / "cb_grad_hist_step_7.pt"
    assert path.exists()
    d = torch.load(path, weights_only=True)
    assert sorted(d) == sorted(["hist", "bin_edges", "bin_centers", "bin_width", "range", "num_bins", "num_samples"])
    assert torch.equal(d["hist"], counts.float())
    assert torch.equal(d["bin_edges"], torch.tensor([-1.0, -0.5, 0.0, 0.5, 1.0]))
    assert torch.equal(d["bin_centers"], torch.tensor([-0.75, -0.25, 0.25, 0.75]))
    assert d["bin_width"] == 0.5 and d["range"] == (-1.0, 1.0) and d["num_bins"] == 4 and d["num_samples"] == 10


def test_dump_refusals(tmp_path):
    c = torch.ones(4)
    with pytest.raises(ValueError):
        quantization.save_distribution_histogram_pt_from_counts(c, None, "s", 1)
    with pytest.raises(ValueError):
        quantization.save_distribution_histogram_pt_from_counts(torch.ones(2, 2), str(tmp_path / "p"), "s", 1)
    with pytest.raises(ValueError):
        quantization.save_distribution_histogram_pt_from_counts(torch.ones(0), str(tmp_path / "p"), "s", 1)
    with pytest.raises(ValueError):
        quantization.save_distribution_histogram_pt_from_counts(c, str(tmp_path / "p"), "s", -1)
    assert not os.listdir(tmp_path)
