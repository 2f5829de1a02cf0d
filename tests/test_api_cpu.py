"""Host-side API checks (CPU only): the reference's public names, argument
validation, and that nothing silently computes on the CPU."""
import pytest
import torch

import cron_root_attention as cra

REFERENCE_ALL = ["cron_root_attention", "cron_root_attention_v14", "cron_root_attention_varlen",
                 "warmup_varlen_shapes", "CronRootAttention", "CronRootMultiheadAttention",
                 "cron_root_attention_hybrid", "CronRootAttentionHybrid", "calibrate",
                 "get_num_sms", "get_gpu_info", "GPU_SM_MAP", "__version__"]


def test_public_names_match_reference():
    assert sorted(cra.__all__) == sorted(REFERENCE_ALL)
    for n in REFERENCE_ALL:
        assert hasattr(cra, n), n
    assert cra.cron_root_attention is cra.cron_root_attention_v14


def test_cpu_tensors_take_the_native_cpu_path():
    """CPU tensors are computed by the library's host code (the reference's
    CPU dispatch, core.py:3794-3796), not refused and not by the oracle."""
    q = torch.randn(1, 2, 64, 32)
    out = cra.cron_root_attention(q, q, q)
    assert out.shape == q.shape and out.dtype == q.dtype and bool(torch.isfinite(out).all())


@pytest.mark.parametrize("shapes,kw,exc", [
    (((1, 2, 64, 32), (1, 2, 63, 32)), {}, ValueError),
    (((1, 3, 64, 32), (1, 2, 64, 32)), {}, ValueError),            # H_q not a multiple of H_kv
    (((2, 64, 32), (2, 64, 32)), {}, ValueError),
])
def test_shape_validation(shapes, kw, exc):
    q = torch.randn(*shapes[0])
    k = torch.randn(*shapes[1])
    with pytest.raises(exc):
        cra.cron_root_attention(q, k, k, **kw)


def test_cpu_path_infers_kv_groups_from_shapes():
    """As the reference's CPU path (cpu_reference.py:219-223): GQA from the
    shapes, the kv_groups argument ignored (the GPU path validates it)."""
    q = torch.randn(1, 4, 64, 32)
    k = torch.randn(1, 2, 64, 32)
    a = cra.cron_root_attention(q, k, k)
    assert torch.equal(a, cra.cron_root_attention(q, k, k, kv_groups=3))
    assert torch.equal(a, cra.cron_root_attention(q, k.repeat_interleave(2, 1),
                                                  k.repeat_interleave(2, 1)))


def test_dtype_validation():
    q = torch.randn(1, 1, 8, 32, dtype=torch.float64)
    with pytest.raises(TypeError):
        cra.cron_root_attention(q, q, q)
    k = torch.randn(1, 1, 8, 32, dtype=torch.float16)
    with pytest.raises(TypeError):
        cra.cron_root_attention(q.float(), k, k)


def test_varlen_validates_boundaries():
    q = torch.randn(1, 2, 100, 32)
    with pytest.raises(ValueError):
        cra.cron_root_attention_varlen(q, q, q, [0, 50, 99])
    with pytest.raises(ValueError):
        cra.cron_root_attention_varlen(q, q, q, [0, 60, 50, 100])


def test_hybrid_below_threshold_is_sdpa_on_any_device():
    q = torch.randn(1, 2, 64, 32)
    out = cra.cron_root_attention_hybrid(q, q, q, backend="auto", threshold=1024)
    ref = torch.nn.functional.scaled_dot_product_attention(q, q, q, is_causal=True)
    assert torch.equal(out, ref)
    assert torch.equal(cra.cron_root_attention_hybrid(q, q, q, backend="cron_root"),
                       cra.cron_root_attention(q, q, q))
    with pytest.raises(ValueError):
        cra.cron_root_attention_hybrid(q, q, q, backend="flash")


def test_module_hybrid_flag_routes_short_sequences_to_sdpa():
    torch.manual_seed(0)
    m = cra.CronRootAttention(d_model=64, n_heads=2, n_kv_heads=1, hybrid=True, threshold=128)
    x = torch.randn(1, 32, 64)
    y = m(x)
    assert y.shape == x.shape
    m2 = cra.CronRootAttention(d_model=64, n_heads=2, hybrid=False)
    assert m2(x).shape == x.shape          # CPU path of the sqrt(N) op


def test_head_dim_limit():
    from cron_root_attention.core import _padded_head_dim
    assert ([_padded_head_dim(d) for d in (1, 16, 32, 33, 64, 65, 128, 129, 200, 256)]
            == [32, 32, 32, 64, 64, 128, 128, 256, 256, 256])
    with pytest.raises(NotImplementedError):
        _padded_head_dim(257)


def test_gpu_info_without_gpu():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    assert cra.get_gpu_info() == {"gpu_name": "No GPU", "sm_count": 0, "is_known_gpu": False}
    assert cra.get_num_sms() == 1


def test_crossover_table_lookup():
    from cron_root_attention.hybrid import CROSSOVER_GFX950, _SDPA_THRESHOLD, crossover
    # measured rows are returned as measured
    for (mode, d, bh), s in CROSSOVER_GFX950.items():
        assert crossover(d, mode == "train", bh) == s
    # larger B*H uses the largest measured row not above it; smaller falls back to the first
    assert crossover(128, True, 4096) == CROSSOVER_GFX950[("train", 128, 64)]
    assert crossover(128, False, 8) == CROSSOVER_GFX950[("fwd", 128, 1)]
    # nearest head dim
    assert crossover(112, True, 16) == CROSSOVER_GFX950[("train", 128, 1)]
    assert crossover(32, False, 16) == CROSSOVER_GFX950[("fwd", 64, 1)]
    assert _SDPA_THRESHOLD == CROSSOVER_GFX950[("train", 128, 1)]
    # the sweep found no crossover: detail says so
    info = crossover(128, True, 64, detail=True)
    assert info["S"] == CROSSOVER_GFX950[("train", 128, 64)] and info["bracketed"] is False
    assert "no crossover" in info["meaning"]
    # more parallel work never raises the crossover
    for mode in ("fwd", "train"):
        for d in (64, 128):
            seq = [crossover(d, mode == "train", bh) for bh in (1, 16, 64, 1024)]
            assert seq == sorted(seq, reverse=True)


def test_hybrid_defaults_use_the_measured_table():
    import inspect
    from cron_root_attention.hybrid import crossover, dispatch_backend
    assert inspect.signature(cra.cron_root_attention_hybrid).parameters["threshold"].default is None
    assert cra.CronRootAttentionHybrid(64, 2).threshold is None
    # config 5 (B*H = 64, D = 128): the gfx950 training crossover, not the static 1536
    thr = crossover(128, True, 64)
    assert thr < 1536
    assert dispatch_backend(thr - 1, 128, True, 64) == "sdpa"
    assert dispatch_backend(thr, 128, True, 64) == "cron_root"
    assert dispatch_backend(1024, 128, True, 64, threshold=1536) == "sdpa"
    assert dispatch_backend(1536, 128, True, 64, threshold=1536) == "cron_root"
    m = cra.CronRootAttention(d_model=64, n_heads=2, hybrid=True, threshold=128)
    assert m.backend_for(torch.zeros(1, 127, 64)) == "sdpa"
    assert m.backend_for(torch.zeros(1, 128, 64)) == "cron_root"
    assert cra.CronRootAttention(64, 2).backend_for(torch.zeros(1, 8, 64)) == "cron_root"


def test_multihead_attention_self_attention_only_both_layouts():
    m = cra.CronRootMultiheadAttention(64, 2, batch_first=False)
    x = torch.randn(16, 1, 64)
    with pytest.raises(AssertionError):
        m(x, x.clone(), x)
    # the same tensor passes the self-attention check in (S, B, E) layout
    out, w = m(x, x, x)
    assert out.shape == x.shape and w is None
