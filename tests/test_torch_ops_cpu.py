"""torch.ops.tq4 registrations (no GPU): schemas with their mutation
annotations, the fake implementations' outputs under meta tensors, and no CPU
implementation (a CPU call raises instead of computing anywhere but the HIP
kernels)."""
import pytest
import torch


@pytest.fixture(scope="module")
def ops(tq4):
    return torch.ops.tq4


def test_schemas_and_mutations(ops):
    pa = str(ops.paged_attention.default._schema)
    assert "Tensor(a7!) workspace" in pa and pa.endswith("-> Tensor")
    for name in ("reshape_and_cache", "reshape_scatter"):
        s = str(getattr(ops, name).default._schema)
        assert "Tensor(a2!) key_cache" in s and "Tensor(a3!) value_cache" in s
        assert "Tensor(a4!) scale_cache" in s and s.endswith("-> ()")


def meta(*shape, dtype=torch.float32):
    return torch.empty(*shape, dtype=dtype, device="meta")


@pytest.mark.parametrize("B,Hq,Hkv,d", [(1, 32, 8, 128), (3, 12, 2, 64), (2, 16, 4, 256)])
def test_fake_paged_attention_shape(ops, B, Hq, Hkv, d):
    q = meta(B, Hq, d, dtype=torch.bfloat16)
    kc = meta(40, Hkv, 16, d // 2, dtype=torch.int8)
    out = ops.paged_attention(q, kc, kc, meta(2, 40, Hkv, 16), meta(B, 9, dtype=torch.int32),
                              meta(B, dtype=torch.int32), meta(d), meta(4096, dtype=torch.uint8),
                              None, Hkv, 16, 0, 0.0, 0.0, 1, False)
    assert out.shape == (B, Hq, d) and out.dtype == torch.bfloat16 and out.device.type == "meta"


def test_fake_writers_return_nothing(ops):
    k = meta(32, 8, 128, dtype=torch.bfloat16)
    kc = meta(64, 8, 16, 64, dtype=torch.int8)
    assert ops.reshape_and_cache(k, k, kc, kc, meta(2, 64, 8, 16), meta(32, dtype=torch.int32),
                                 meta(128), None, 16, 0.0) is None
    assert ops.reshape_scatter(k, k, kc, kc, meta(2, 64, 8, 16), meta(32, dtype=torch.int32),
                               meta(128), None, 16, 0.0) is None


def test_cpu_tensors_raise(ops):
    q = torch.zeros(1, 8, 128, dtype=torch.bfloat16)
    kc = torch.zeros(4, 2, 16, 64, dtype=torch.int8)
    with pytest.raises(NotImplementedError):
        ops.paged_attention(q, kc, kc, torch.zeros(2, 4, 2, 16), torch.zeros(1, 4, dtype=torch.int32),
                            torch.ones(1, dtype=torch.int32), torch.ones(128),
                            torch.zeros(64, dtype=torch.uint8), None, 2, 16, 1, 0.0, 0.0, 1, False)


def test_kv4fp8_schemas_and_fakes(ops):
    s = str(ops.fused_decode_opt.default._schema)
    assert "Tensor(a6!) workspace" in s and s.endswith("-> Tensor")
    r = str(ops.fused_decode_opt_raw_query.default._schema)
    assert "Tensor(a3!) query_rot" in r and "Tensor(a9!) workspace" in r
    T, Hq, H, S = 2, 32, 2, 64
    kc = meta(10 * S * H * 128, dtype=torch.uint8)
    args = (kc, kc, meta(10 * S * 8), meta(T, 5, dtype=torch.int32), meta(T, dtype=torch.int32),
            meta(4096, dtype=torch.uint8))
    for bf16 in (False, True):
        out = ops.fused_decode_opt(meta(T, Hq, 256), *args, H, S, 1, 16, 4096, 0.0, 0.0, bf16)
        assert out.shape == (T, Hq, 256) and out.device.type == "meta"
        assert out.dtype == (torch.bfloat16 if bf16 else torch.float16)
    q = meta(T, Hq, 256, dtype=torch.bfloat16)
    out = ops.fused_decode_opt_raw_query(q, meta(256), None, meta(T, Hq, 256), *args, H, S, 1,
                                         16, 1, 4096, 0.0, 0.0)
    assert out.shape == q.shape and out.dtype == torch.bfloat16


def test_kv4fp8_cpu_tensors_raise(ops):
    kc = torch.zeros(4 * 64 * 128, dtype=torch.uint8)
    with pytest.raises(NotImplementedError):
        ops.fused_decode_opt(torch.zeros(1, 16, 256), kc, kc, torch.ones(4 * 64 * 8),
                             torch.zeros(1, 4, dtype=torch.int32), torch.ones(1, dtype=torch.int32),
                             torch.zeros(4096, dtype=torch.uint8), 1, 64, 1, 16, 4096, 0.0, 0.0,
                             False)
