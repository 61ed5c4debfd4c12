"""Host <-> device helpers for the GPU parity tests (numpy <-> torch)."""
import numpy as np
import torch

from oracle_bindings import bf16_to_f32

DEV = torch.device("cuda:0")
CANARY_WORD = 0x7FC0BEEF  # quiet-NaN canary of the reference rigs


def dev(a):
    """numpy -> device tensor; uint16 arrays become bfloat16 tensors (same bits)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(DEV).view(torch.bfloat16)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).to(DEV)
    return torch.from_numpy(a).to(DEV)


def host(t):
    """device tensor -> numpy; bfloat16 comes back as uint16 bits."""
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def canary_bytes(n):
    """n bytes of the 0x7FC0BEEF canary pattern (int8)."""
    words = np.full((n + 3) // 4, CANARY_WORD, np.uint32)
    return words.view(np.int8)[:n].copy()


def canary_floats(n):
    return np.full(n, CANARY_WORD, np.uint32).view(np.float32).copy()


def bf16_out_error(got_bits, want_f32):
    """(max-abs, mean-rel) of a BF16 output against an FP32 reference rounded to BF16."""
    from oracle_bindings import f32_to_bf16
    got = bf16_to_f32(got_bits).astype(np.float64)
    want = bf16_to_f32(f32_to_bf16(want_f32)).astype(np.float64)
    diff = np.abs(got - want)
    return float(diff.max()), float(diff.sum() / max(np.abs(want).sum(), 1e-30))


# (label, max-abs, mean-rel, max-abs budget, mean-rel budget) of every decode
# output compared; conftest prints them as fractions of the budget at the end
# of the session, the way the reference rig reports its margins
# (tests/npu/turboquant_splitk_rigs.hpp:103-215).
MARGINS = []


def record_margin(label, mx, mr, mx_budget, mr_budget):
    MARGINS.append((str(label), float(mx), float(mr), float(mx_budget), float(mr_budget)))
