"""The reference's own test suite (tests/test_attention.py:26-200), restated
for this build: same shapes, same API calls, same assertions."""
import time

import pytest
import torch

pytestmark = pytest.mark.gpu

device = torch.device("cuda")
dtype = torch.float16


class TestCronRootAttention:
    def test_import(self):
        from cron_root_attention import (GPU_SM_MAP, CronRootAttention, CronRootMultiheadAttention,
                                         cron_root_attention, get_gpu_info)
        assert callable(cron_root_attention) and callable(get_gpu_info)

    def test_forward_shape(self):
        from cron_root_attention import cron_root_attention
        B, H, S, D = 2, 4, 256, 64
        q, k, v = (torch.randn(B, H, S, D, device=device, dtype=dtype) for _ in range(3))
        out = cron_root_attention(q, k, v)
        assert out.shape == (B, H, S, D) and out.dtype == dtype

    def test_no_nan_inf(self):
        from cron_root_attention import cron_root_attention
        q, k, v = (torch.randn(1, 8, 512, 64, device=device, dtype=dtype) for _ in range(3))
        out = cron_root_attention(q, k, v)
        assert not torch.isnan(out).any() and not torch.isinf(out).any()

    def test_backward_shape(self):
        from cron_root_attention import cron_root_attention
        q, k, v = (torch.randn(1, 2, 128, 32, device=device, dtype=torch.float32,
                               requires_grad=True) for _ in range(3))
        cron_root_attention(q, k, v).sum().backward()
        for t in (q, k, v):
            assert t.grad is not None and t.grad.shape == t.shape

    def test_backward_no_nan(self):
        from cron_root_attention import cron_root_attention
        q, k, v = (torch.randn(1, 2, 256, 32, device=device, dtype=torch.float32,
                               requires_grad=True) for _ in range(3))
        out = cron_root_attention(q, k, v)
        out.backward(torch.randn_like(out))
        for t in (q, k, v):
            assert not torch.isnan(t.grad).any()

    def test_module_api(self):
        from cron_root_attention import CronRootAttention
        attn = CronRootAttention(d_model=512, n_heads=8).to(device).to(dtype)
        x = torch.randn(2, 256, 512, device=device, dtype=dtype)
        assert attn(x).shape == (2, 256, 512)

    def test_multihead_attention_api(self):
        from cron_root_attention import CronRootMultiheadAttention
        mha = CronRootMultiheadAttention(embed_dim=512, num_heads=8, batch_first=True)
        mha = mha.to(device).to(dtype)
        x = torch.randn(2, 256, 512, device=device, dtype=dtype)
        out, w = mha(x, x, x)
        assert out.shape == (2, 256, 512) and w is None

    def test_gpu_info(self):
        from cron_root_attention import get_gpu_info
        info = get_gpu_info()
        assert {"gpu_name", "sm_count", "is_known_gpu"} <= set(info)
        assert info["sm_count"] > 0

    def test_hybrid_backend(self):
        from cron_root_attention import cron_root_attention_hybrid
        q, k, v = (torch.randn(1, 4, 2048, 64, device=device, dtype=dtype) for _ in range(3))
        for backend in ("auto", "cron_root", "sdpa"):
            assert cron_root_attention_hybrid(q, k, v, backend=backend).shape == (1, 4, 2048, 64)


class TestCronRootScaling:
    def test_complexity_scaling(self):
        from cron_root_attention import cron_root_attention
        times = {}
        for S in (1024, 4096):
            q, k, v = (torch.randn(1, 4, S, 64, device=device, dtype=dtype) for _ in range(3))
            for _ in range(3):
                cron_root_attention(q, k, v)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(10):
                cron_root_attention(q, k, v)
            torch.cuda.synchronize()
            times[S] = (time.perf_counter() - t0) / 10
        assert times[4096] / times[1024] < 16


def test_module_gqa_and_hybrid_flag():
    from cron_root_attention import CronRootAttention
    torch.manual_seed(0)
    m = CronRootAttention(d_model=256, n_heads=4, n_kv_heads=2, hybrid=True, threshold=512)
    m = m.to(device).to(dtype)
    for S in (256, 3000):
        x = torch.randn(1, S, 256, device=device, dtype=dtype, requires_grad=True)
        y = m(x)
        y.float().sum().backward()
        assert y.shape == x.shape and torch.isfinite(x.grad).all()


def test_varlen_equals_per_document_calls():
    from cron_root_attention import cron_root_attention, cron_root_attention_varlen
    torch.manual_seed(1)
    cu = [0, 700, 3000, 3100]
    q, k, v = (torch.randn(1, 2, 3100, 64, device=device, dtype=dtype) for _ in range(3))
    out = cron_root_attention_varlen(q, k, v, torch.tensor(cu))
    for s, e in zip(cu, cu[1:]):
        ref = cron_root_attention(q[:, :, s:e].contiguous(), k[:, :, s:e].contiguous(),
                                  v[:, :, s:e].contiguous())
        assert torch.equal(out[:, :, s:e], ref)


def test_calibrate_and_warmup():
    import cron_root_attention as cra
    cfg = cra.calibrate(H=2, D=64, S=1024, verbose=False)
    assert set(cfg) == {"fwd", "bwd"}
    cra.warmup_varlen_shapes([100, 2500], H=2, D=64)
