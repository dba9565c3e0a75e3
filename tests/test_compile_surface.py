"""The torch.compile surface on the host (no GPU): the reference's custom-op
names and mutation contracts (kernels/automatic_gefen_fused.py:447-490,
kernels/period_variance.py:36-57), fake-tensor propagation, and that a traced
call of a public wrapper on the capturable entry stays one graph with the op
inside it."""
import pytest
import torch

import gefen  # noqa: F401  (registers the ops)
from gefen.kernels import automatic_gefen_fused as fused

# op -> arguments it mutates (the reference's mutates_args)
EXPECTED = {
    "fused_full_update": {"p", "m_sign", "m_magnitude", "vmean"},
    "factored_update": {"p", "m_sign", "m_magnitude", "v_row", "v_col"},
    "quantized_momentum_update": {"m_sign", "m_magnitude", "momentum_out"},
    "fused_update_v2_full": {"p", "m_sign", "m_magnitude", "vmean"},
    "average_within_block_variance_cuda": set(),
}


@pytest.mark.parametrize("name", sorted(EXPECTED))
def test_op_registered_with_reference_mutations(name):
    assert fused._COMPILE_OPS_REGISTERED
    schema = getattr(torch.ops.gefen, name).default._schema
    mutated = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
    assert mutated == EXPECTED[name], (name, mutated)


def _factored_args(rows=8, cols=16, period=32):
    nb = rows * cols // period
    return dict(
        p=torch.zeros(rows, cols, dtype=torch.bfloat16), grad_view=torch.zeros(nb, period, dtype=torch.bfloat16),
        m_sign=torch.zeros(nb, period, dtype=torch.uint8), m_magnitude=torch.zeros(nb, 1),
        v_row=torch.zeros(rows), v_col=torch.zeros(cols), codebook=torch.linspace(-1, 1, 16), cols=cols,
        beta1=0.9, beta2=0.999, lr=1e-3, eps=1e-8, inv_bias_correction_2=1.0, inv_bias_correction_1=1.0,
        weight_decay_factor=1.0, stochastic_round=False, rng_seed=0, step_scalars=torch.ones(4),
        codebook_lut=torch.zeros(4097, dtype=torch.int16), seed_dev=None)


def test_fake_propagation_runs_no_kernel():
    from torch._subclasses.fake_tensor import FakeTensorMode
    args = _factored_args()
    with FakeTensorMode() as mode:
        fake = {k: (mode.from_tensor(v) if torch.is_tensor(v) else v) for k, v in args.items()}
        assert torch.ops.gefen.factored_update(**fake) is None
        out = torch.ops.gefen.average_within_block_variance_cuda(fake["p"].reshape(-1), 32, False)
        assert out.shape == () and out.dtype == torch.float32


def test_traced_wrapper_is_one_graph_holding_the_op():
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)
        return lambda *a: None  # tracing only: nothing runs on the host tensors

    def step(a):
        fused.gefen_factored_update_cuda(**a)

    torch._dynamo.reset()
    torch.compile(step, backend=backend, fullgraph=True)(_factored_args())
    torch._dynamo.reset()
    assert len(graphs) == 1
    targets = [str(n.target) for n in graphs[0].graph.nodes if n.op == "call_function"]
    assert any("gefen.factored_update" in t for t in targets), targets


def test_eager_default_path_skips_the_op():
    """Outside tracing, and on the non-capturable entry, the wrapper calls the
    implementation directly (its host checks run: a host tensor is refused)."""
    args = _factored_args()
    args["step_scalars"] = None
    with pytest.raises(ValueError, match="HIP device"):
        fused.gefen_factored_update_cuda(**args)


def test_every_kernel_name_the_reference_optimizer_imports_resolves():
    """The names gefen.py imports from the kernel modules (gefen.py:25-51,
    the lazy histogram import at 444-446, partitioning.py:216) resolve here,
    without a GPU (the library is loaded on first call)."""
    import importlib
    names = {
        "gefen.partitioning": ["find_period_by_block_variance"],
        "gefen.kernels.automatic_vmean": ["automatic_vmean_update_cuda", "_load_extension"],
        "gefen.kernels.automatic_gefen_fused": [
            "automatic_gefen_fused_update_cuda", "automatic_gefen_fused_full_update_cuda",
            "automatic_gefen_fused_update_v2_full_cuda", "gefen_quantized_momentum_update_cuda",
            "gefen_factored_update_cuda", "_should_use_v2_full", "_should_use_v2", "_CAPT_V1_FULL_TINY_NUMEL",
            "_codebook_search_lut", "ensure_extension_loaded", "_load_extension"],
        "gefen.kernels.exact_histogram_fused": ["gefen_exact_histogram_cuda", "_load_extension"],
        "gefen.kernels.period_variance": ["average_within_block_variance_cuda_kernel"],
    }
    for mod, attrs in names.items():
        m = importlib.import_module(mod)
        for a in attrs:
            assert hasattr(m, a), "%s.%s" % (mod, a)
