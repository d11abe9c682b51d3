"""Input builders shared by the CPU and GPU tests.

The builders reproduce the inputs of the reference's own tests (same seeds,
same draw order), so the parity tests read like tests/test_*.py upstream.
"""

from __future__ import annotations

import numpy as np
import torch


def cu_list(lengths):
    out = [0]
    for n in lengths:
        out.append(out[-1] + n)
    return out


def cu_tensor(lengths, device="cpu"):
    return torch.tensor(cu_list(lengths), dtype=torch.int32, device=device)


def attention_inputs(lengths, groups, ratio, dimension, block_size, topk):
    """tests/test_triton_attention.py:35-55: bf16 q/k/v from seed 1234 and
    deterministic distinct selections (current block first, then every other
    earlier block offset by group). Returns CPU tensors."""
    generator = torch.Generator().manual_seed(1234)
    total = sum(lengths)
    q = torch.randn(total, groups * ratio, dimension, generator=generator).to(torch.bfloat16)
    k = torch.randn(total, groups, dimension, generator=generator).to(torch.bfloat16)
    v = torch.randn(total, groups, dimension, generator=generator).to(torch.bfloat16)
    cu = cu_tensor(lengths)
    indices = torch.full((total, groups, topk), -1, dtype=torch.int32)
    start = 0
    for length in lengths:
        for offset in range(length):
            for group in range(groups):
                current_block = offset // block_size
                candidates = [current_block]
                candidates += [b for b in range(current_block) if (b + group) % 2 == 0]
                chosen = candidates[:topk]
                if chosen:
                    indices[start + offset, group, : len(chosen)] = torch.tensor(chosen, dtype=torch.int32)
        start += length
    return (q, k, v), indices, cu


def np64(x):
    return x.detach().cpu().double().numpy()


def random_selection(total, groups, topk, lengths, block_size, local_blocks, generator):
    """Random distinct causal selections with the local blocks forced, like m3_topk output."""
    ids = torch.full((total, groups, topk), -1, dtype=torch.int32)
    start = 0
    rng = np.random.default_rng(int(torch.randint(0, 2**31 - 1, (1,), generator=generator)))
    for length in lengths:
        for pos in range(length):
            qb = pos // block_size
            forced = list(range(qb, max(-1, qb - local_blocks), -1))
            pool = np.arange(0, max(0, qb - local_blocks + 1))
            extra = min(topk - len(forced), pool.size)
            picks = rng.choice(pool, size=extra, replace=False).tolist() if extra > 0 else []
            chosen = (forced + picks)[:topk]
            for g in range(groups):
                if g:
                    picks_g = rng.choice(pool, size=extra, replace=False).tolist() if extra > 0 else []
                    chosen = (forced + picks_g)[:topk]
                ids[start + pos, g, : len(chosen)] = torch.tensor(chosen, dtype=torch.int32)
        start += length
    return ids


def rounded(x, dtype):
    """FP64 oracle values in `dtype`, rounded as the kernels round their FP64 results:
    float32 and float16 once (numpy's direct casts), bfloat16 through float32 (as the
    reference's fp32 kernels followed by a bf16 cast, and torch's float64 -> bfloat16
    cast). torch's float64 -> float16 cast also goes through float32; a value just past
    a float16 midpoint then lands on it and rounds to even, numpy's cast does not."""
    x = np.asarray(x, dtype=np.float64)
    if dtype == torch.float64:
        return torch.from_numpy(x.copy())
    if dtype == torch.float32:
        return torch.from_numpy(x.astype(np.float32))
    if dtype == torch.float16:
        return torch.from_numpy(x.astype(np.float16))
    assert dtype == torch.bfloat16, dtype
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)


def check_bf16_stated(actual, expected, what):
    """The stated bf16 tolerance for large outputs: every element within 1e-4 + 2^-8 |x|
    of the FP64 value x, and at most 0.1 % (at least one) outside the reference's gate
    (atol = rtol = 1e-4 after rounding x to bf16). fp32 arithmetic leaves values within
    ~2^-22 of a bf16 rounding midpoint undecided, ~5e-5 of the elements here."""
    act = actual.detach().float().cpu().numpy().astype(np.float64).ravel()
    exp = np.asarray(expected, dtype=np.float64).ravel()
    ref_r = rounded(exp, torch.bfloat16).double().numpy()
    gate = np.abs(act - ref_r) <= 1e-4 + 1e-4 * np.abs(ref_r)
    bad = int((~gate).sum())
    err = np.abs(act - exp)
    bound = 1e-4 + 2.0 ** -8 * np.abs(exp)
    worst = np.argsort(-(err / bound))[:5]
    detail = ", ".join(f"(got {act[i]:.6g}, fp64 {exp[i]:.6g})" for i in worst)
    print(f"{what}: {bad} of {gate.size} outside the 1e-4 gate; worst err/bound {float((err / bound).max()):.3f}: "
          f"{detail}", flush=True)
    assert bad <= max(1, gate.size // 1000), f"{what}: {bad} of {gate.size} elements outside the gate; {detail}"
    assert np.all(err <= bound), f"{what}: error above 1e-4 + 2^-8 |x|; {detail}"
