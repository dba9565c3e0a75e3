"""The reference's large-tensor regressions (tests/test_large_tensor_paths.py
there) on MI355X: the block-variance kernel against a float64 torch
reduction at small sizes (squared or raw input); a 2,440,000,000-element
tensor (more than 2^31) at periods 1, 2 and numel/2; the "gpu" backend of the
period search (squared values) choosing what the "cuda_kernel" backend
chooses on the raw grad; the step-1 codebook learned whole or in block-aligned
chunks, bit-identical."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

HUGE_NUMEL = 2_440_000_000


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _ref_error(values, period):
    v = values.detach().double().cpu().reshape(-1, period)
    return float(v.var(dim=1, correction=0).mean().sqrt())


@pytest.mark.parametrize("input_is_squared", [True, False])
def test_block_variance_matches_a_float64_reduction(dev, input_is_squared):
    from gefen.kernels.period_variance import average_within_block_variance_cuda_kernel
    from gefen.partitioning import average_within_block_variance_torch
    torch.manual_seed(0)
    for n, p in [(1024, 8), (1_000_000, 100), (4_194_304, 256), (999_936, 96)]:
        x = torch.rand(n, device=dev, dtype=torch.float32) + 0.1
        got = average_within_block_variance_cuda_kernel(x, p, input_is_squared=input_is_squared)
        sq = x if input_is_squared else x * x
        assert got == pytest.approx(_ref_error(sq, p), rel=1e-5), (n, p)
        assert average_within_block_variance_torch(sq, p) == pytest.approx(_ref_error(sq, p), rel=1e-5)


def test_block_variance_of_more_than_2_31_elements(dev):
    from gefen.kernels.period_variance import average_within_block_variance_cuda_kernel
    free, _ = torch.cuda.mem_get_info()
    if free < HUGE_NUMEL * 2 * 1.2:
        pytest.skip("needs ~5.5 GiB free")
    print("variance of %d elements" % HUGE_NUMEL, flush=True)
    x = torch.rand(HUGE_NUMEL, device=dev, dtype=torch.bfloat16)
    for period in (1, 2, HUGE_NUMEL // 2):
        assert math.isfinite(average_within_block_variance_cuda_kernel(x, period, input_is_squared=True))
    del x
    torch.cuda.empty_cache()


def test_period_search_backends_agree(dev):
    from gefen import partitioning
    torch.manual_seed(1)
    g = (torch.randn(96, 384, device=dev) * torch.linspace(0.1, 3.0, 384, device=dev)).reshape(-1)
    a = partitioning.find_period_by_block_variance(g * g, print_results=False, backend="gpu")
    b = partitioning.find_period_by_block_variance(g, print_results=False, backend="cuda_kernel",
                                                  input_is_squared=False)
    c = partitioning.find_period_by_block_variance(g * g, print_results=False, backend="cuda_kernel",
                                                  input_is_squared=True)
    assert a == b == c


def test_codebook_from_whole_or_chunked_histogram_is_identical(dev, monkeypatch):
    import gefen.gefen as gefen_mod
    torch.manual_seed(0)
    period = 96
    flat = torch.randn(4096 * period, device=dev, dtype=torch.bfloat16) * 1e-3
    kw = dict(grad_periods=[("w", flat, period, None)], codebook_device=dev, num_codebooks=16,
              force_endpoints=False, verbose=False, compute_mse_logging=False)
    whole = gefen_mod.learn_gefen_exact_codebook_from_grad_periods(**kw)
    monkeypatch.setattr(gefen_mod, "GEFEN_EXACT_HISTOGRAM_CHUNK", 5 * period)
    chunked = gefen_mod.learn_gefen_exact_codebook_from_grad_periods(**kw)
    assert whole.numel() == 16 and torch.equal(whole, chunked)
