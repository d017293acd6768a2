"""Host-side argument checks of the kernel wrappers: inputs that are not on a
GPU (or of the wrong dtype or size) raise before any launch, so no host
pointer or short buffer ever reaches a kernel.  No GPU needed."""
import pytest
import torch

from specdec import ops


def test_cpu_inputs_are_rejected_before_launch():
    v = 16
    p = torch.rand(1, 5, v)
    q = torch.rand(1, 4, v)
    draft = torch.zeros(1, 4, dtype=torch.int64)
    u = torch.rand(1, 4)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.probabilities(torch.randn(3, v), 1.0)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.accept_reject(p, q, draft, u, torch.rand(1))
    with pytest.raises(RuntimeError, match="GPU"):
        ops.accept_count(p, q, draft, u)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.sample_inverse_cdf(torch.rand(2, v), torch.rand(2))
    with pytest.raises(RuntimeError, match="GPU"):
        ops.ngram_lookup(torch.zeros(2, 8, dtype=torch.int32), torch.full((2,), 8, dtype=torch.int32), 4, 3)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.block_plan(torch.zeros(2, 4, dtype=torch.int32), torch.zeros(8, dtype=torch.int32),
                       torch.zeros(8, dtype=torch.uint8), 8, torch.zeros(4, dtype=torch.int32), 1, 0)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.add_rmsnorm(torch.randn(2, 8), None, torch.ones(8), torch.empty(2, 8), 1e-5)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.silu_mul(torch.randn(2, 8), torch.empty(2, 4))
    with pytest.raises(RuntimeError, match="GPU"):
        ops.rms_silu_mul(torch.randn(2, 8), torch.randn(2, 6), torch.empty(2, 4), 1e-5)


def test_checker_names_device_dtype_and_size():
    t = torch.zeros(4, dtype=torch.int32)
    assert ops._on(t.device, t, "t", torch.int32, True, 4) is t
    with pytest.raises(TypeError, match="int64"):
        ops._on(t.device, t, "t", torch.int64)
    with pytest.raises(ValueError, match="5 elements"):
        ops._on(t.device, t, "t", numel=5)
    with pytest.raises(ValueError, match="contiguous"):
        ops._on(t.device, torch.zeros(4, 4)[:, 0], "t", contiguous=True)
    with pytest.raises(RuntimeError, match="must be on"):
        ops._on(torch.device("meta"), t, "t")


def test_tile_weight_layout():
    """ops.tile_weight puts W[n, k] at ((n // 16 * (K // 32) + k // 32) * 64
    + (k % 32) // 8 * 16 + n % 16) * 8 + k % 8, the layout the C ABI documents
    (SPECDEC_W_TILED): every element checked by its index."""
    n, k = 48, 96
    w = torch.arange(n * k, dtype=torch.float32).reshape(n, k)
    flat = ops.tile_weight(w).reshape(-1)
    nn, kk = torch.meshgrid(torch.arange(n), torch.arange(k), indexing="ij")
    pos = ((nn // 16 * (k // 32) + kk // 32) * 64 + (kk % 32) // 8 * 16 + nn % 16) * 8 + kk % 8
    assert torch.equal(flat[pos.reshape(-1)], w.reshape(-1))
    with pytest.raises(ValueError):
        ops.tile_weight(torch.zeros(40, 96))
