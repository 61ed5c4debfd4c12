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
