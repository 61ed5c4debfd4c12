"""The host mirror's operand checks (no GPU): a dtype or size the kernels
would misread is refused with ValueError before anything is launched, both
through the Python entry points and the torch.ops.tq4 operators. Correctly
typed host tensors get past the checks and are then refused for not being on
the device, which shows the checks do not reject valid operands."""
import pytest
import torch

B, HQ, HKV, D, S, P, MAXB = 2, 8, 2, 128, 16, 12, 5


def decode_args(**over):
    a = dict(q=torch.zeros(B, HQ, D, dtype=torch.bfloat16),
             key_cache=torch.zeros(P * HKV * S * D // 2, dtype=torch.int8),
             value_cache=torch.zeros(P * HKV * S * D // 2, dtype=torch.int8),
             scale_cache=torch.zeros(2 * P * HKV * S, dtype=torch.float32),
             block_tables=torch.zeros(B, MAXB, dtype=torch.int32),
             context_lens=torch.zeros(B, dtype=torch.int32),
             pi_signs=torch.ones(D, dtype=torch.float32))
    a.update(over)
    return a


def call_decode(tq4, gate=None, out=None, **over):
    a = decode_args(**over)
    return tq4.paged_decode(a["q"], a["key_cache"], a["value_cache"], a["scale_cache"],
                            a["block_tables"], a["context_lens"], a["pi_signs"], HKV, S, P,
                            gate=gate, out=out, output_stage=2 if gate is not None else 1)


@pytest.mark.parametrize("over,match", [
    (dict(q=torch.zeros(B, HQ, D, dtype=torch.float16)), "q must be bfloat16"),
    (dict(q=torch.zeros(B * HQ, D, dtype=torch.bfloat16)), "q must have 3 dimensions"),
    (dict(block_tables=torch.zeros(B, MAXB, dtype=torch.int64)), "block_tables must be int32"),
    (dict(block_tables=torch.zeros(B + 1, MAXB, dtype=torch.int32)), "block_tables must have 2 rows"),
    (dict(context_lens=torch.zeros(B, dtype=torch.int64)), "context_lens must be int32"),
    (dict(context_lens=torch.zeros(B + 1, dtype=torch.int32)), "context_lens must hold 2"),
    (dict(scale_cache=torch.zeros(2 * P * HKV * S, dtype=torch.float16)), "scale_cache must be float32"),
    (dict(scale_cache=torch.zeros(P * HKV * S, dtype=torch.float32)), "scale_cache must hold at least"),
    (dict(key_cache=torch.zeros(P * HKV * S * D // 2 - 1, dtype=torch.int8)), "key_cache must hold at least"),
    (dict(value_cache=torch.zeros(P * HKV * S * D // 2, dtype=torch.float32)), "value_cache must be int8"),
    (dict(pi_signs=torch.ones(D, dtype=torch.bfloat16)), "pi_signs must be float32"),
    (dict(pi_signs=None), "pi_signs is required"),
])
def test_paged_decode_refusals(tq4, over, match):
    with pytest.raises(ValueError, match=match):
        call_decode(tq4, **over)


def test_paged_decode_gate_and_out_refusals(tq4):
    with pytest.raises(ValueError, match="gate must be float32"):
        call_decode(tq4, gate=torch.zeros(B, HQ, D, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="gate must hold"):
        call_decode(tq4, gate=torch.zeros(B, HQ, D // 2, dtype=torch.float32))
    with pytest.raises(ValueError, match="out must be bfloat16"):
        call_decode(tq4, out=torch.zeros(B, HQ, D, dtype=torch.float32))


def test_valid_operands_pass_the_checks(tq4):
    """Correct dtypes and sizes reach the device check (host tensors)."""
    with pytest.raises(ValueError, match="must be a device tensor"):
        call_decode(tq4)
    with pytest.raises(ValueError, match="must be a device tensor"):
        call_decode(tq4, gate=torch.zeros(B, HQ, D, dtype=torch.float32))


def test_partials_and_combine_refusals(tq4):
    a = decode_args()
    with pytest.raises(ValueError, match="context_lens must be int32"):
        tq4.paged_decode_partials(a["q"], a["key_cache"], a["value_cache"], a["scale_cache"],
                                  a["block_tables"], a["context_lens"].long(), a["pi_signs"],
                                  HKV, S, P, 4)
    with pytest.raises(ValueError, match="workspace must hold at least"):
        tq4.paged_decode_partials(a["q"], a["key_cache"], a["value_cache"], a["scale_cache"],
                                  a["block_tables"], a["context_lens"], a["pi_signs"], HKV, S,
                                  P, 4, workspace=torch.zeros(10, dtype=torch.float32))
    ws = torch.zeros(B * HQ * 4 * (D + 4), dtype=torch.float32)
    with pytest.raises(ValueError, match="workspace must be float32"):
        tq4.splitk_combine(ws.view(torch.int32), a["pi_signs"], B, HQ, D, 4)
    with pytest.raises(ValueError, match="gate must be float32"):
        tq4.splitk_combine(ws, a["pi_signs"], B, HQ, D, 4, output_stage=2,
                           gate=torch.zeros(B, HQ, D, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="must be a device tensor"):
        tq4.splitk_combine(ws, a["pi_signs"], B, HQ, D, 4)


def writer_args(dtype=torch.bfloat16, tokens=32, **over):
    a = dict(key=torch.zeros(tokens, HKV, D, dtype=dtype),
             value=torch.zeros(tokens, HKV, D, dtype=dtype),
             key_cache=torch.zeros(P * HKV * S * D // 2, dtype=torch.int8),
             value_cache=torch.zeros(P * HKV * S * D // 2, dtype=torch.int8),
             scale_cache=torch.zeros(2 * P * HKV * S, dtype=torch.float32),
             slot_mapping=torch.arange(tokens, dtype=torch.int32),
             pi_signs=torch.ones(D, dtype=torch.float32))
    a.update(over)
    return a


@pytest.mark.parametrize("over,match", [
    (dict(slot_mapping=torch.arange(32, dtype=torch.int64)), "slot_mapping must be int32"),
    (dict(slot_mapping=torch.arange(16, dtype=torch.int32)), "slot_mapping must hold at least 32"),
    (dict(value=torch.zeros(16, HKV, D, dtype=torch.bfloat16)), "value must hold"),
    (dict(pi_signs=torch.ones(D // 2, dtype=torch.float32)), "pi_signs must hold at least"),
    (dict(scale_cache=torch.zeros(2 * P * HKV * S, dtype=torch.float64)), "scale_cache must be float32"),
])
def test_writer_refusals(tq4, over, match):
    a = writer_args(**over)
    with pytest.raises(ValueError, match=match):
        tq4.reshape_and_cache_bf16(**a, num_blocks=P, block_size=S)


def test_writer_tables_dtype(tq4):
    a = writer_args(torch.int8, pi_signs=None)
    with pytest.raises(ValueError, match="tables must be int8"):
        tq4.reshape_and_cache_a8(**a, tables=torch.zeros(64 * D, dtype=torch.bfloat16),
                                 num_blocks=P, block_size=S)
    with pytest.raises(ValueError, match="must be a device tensor"):
        tq4.reshape_and_cache_a8(**a, tables=torch.zeros(64 * D, dtype=torch.int8),
                                 num_blocks=P, block_size=S)


def test_scatter_refusals(tq4):
    a = writer_args()
    with pytest.raises(ValueError, match="cu_seqlens must be int32"):
        tq4.reshape_scatter(**a, cu_seqlens=torch.tensor([0, 32], dtype=torch.int64),
                            num_blocks=P, block_size=S)
    with pytest.raises(ValueError, match="need 40 tokens"):
        tq4.reshape_scatter(**a, num_requests=40, num_blocks=P, block_size=S)
    with pytest.raises(ValueError, match="must be a device tensor"):
        tq4.reshape_scatter(**a, num_blocks=P, block_size=S)


def test_kv4fp8_refusals(tq4):
    T, H, G, S4, pages = 1, 1, 16, 128, 4
    P4 = pages
    q = torch.zeros(T, H * G, 256, dtype=torch.float32)
    key = torch.zeros(P4 * S4 * H * 128, dtype=torch.uint8)
    sc = torch.zeros(P4 * S4 * 8, dtype=torch.float32)
    tb = torch.zeros(T, pages, dtype=torch.int32)
    ln = torch.zeros(T, dtype=torch.int32)
    with pytest.raises(ValueError, match="query must be float32"):
        tq4.kv4fp8_decode(q.half(), key, key, sc, tb, ln, H, S4, P4)
    with pytest.raises(ValueError, match="block_table must be int32"):
        tq4.kv4fp8_decode(q, key, key, sc, tb.long(), ln, H, S4, P4)
    with pytest.raises(ValueError, match="scales must hold at least"):
        tq4.kv4fp8_decode(q, key, key, sc[:-1], tb, ln, H, S4, P4)
    raw = torch.zeros(T, H * G, 256, dtype=torch.bfloat16)
    signs = torch.ones(256)
    with pytest.raises(ValueError, match="gate must be bfloat16"):
        tq4.kv4fp8_decode_raw_query(raw, signs, key, key, sc, tb, ln, H, S4, P4,
                                    gate=torch.zeros(raw.shape, dtype=torch.float32),
                                    output_stage=2)
    with pytest.raises(ValueError, match="must be a device tensor"):
        tq4.kv4fp8_decode_raw_query(raw, signs, key, key, sc, tb, ln, H, S4, P4,
                                    gate=torch.zeros(raw.shape, dtype=torch.bfloat16),
                                    output_stage=2)


def test_torch_op_refuses_bad_gate(tq4):
    """tq4::paged_attention's device implementation goes through the same
    checks (a BF16 gate would otherwise be read as twice its bytes of FP32).
    The dispatcher refuses host tensors before any implementation runs, so
    the operator's function is called directly."""
    import sys
    impl = sys.modules["ascend_micro_harness_amd.torch_ops"].paged_attention._init_fn
    a = decode_args()
    with pytest.raises(ValueError, match="gate must be float32"):
        impl(a["q"], a["key_cache"], a["value_cache"], a["scale_cache"],
                            a["block_tables"], a["context_lens"], a["pi_signs"],
                            torch.zeros(4096, dtype=torch.uint8),
                            torch.zeros(B, HQ, D, dtype=torch.bfloat16), HKV, S, 0, 0.0, 0.0, 2,
                            False)
