"""msa_k2q_build_noalloc (the CSR build over the library's fixed per-GPU scratch array)
against msa_k2q_build with a caller workspace: bit-identical row_ptr / query / slot
arrays on two calls in a row, the second with a smaller input (the scratch array keeps
the first call's contents), and a clear refusal of a request beyond the array."""

from __future__ import annotations

import pytest
import torch

from msa_triton_amd import _lib
from msa_triton_amd.layout import sequence_meta
from tests.helpers import cu_list, random_selection

pytestmark = pytest.mark.gpu

NOALLOC_MAX_ELEMS = 1 << 22  # MSA_K2Q_NOALLOC_MAX_ELEMS in include/msa_mi355x.h


def _case(lengths, groups, topk, block, seed, device):
    gen = torch.Generator().manual_seed(seed)
    total = sum(lengths)
    ids = random_selection(total, groups, topk, lengths, block, 1, gen)
    ids[::7, :, -1] = ids[::7, :, 0]  # duplicates stay edges of their own
    ids[::11, :, 1] = -1
    meta = sequence_meta(cu_list(lengths), block)
    cu = torch.tensor(cu_list(lengths), dtype=torch.int32, device=device)
    cbl = torch.tensor(meta.cu_block_lens, dtype=torch.int32, device=device)
    tri = torch.tensor([groups * x for x in meta.tri_prefix], dtype=torch.int64, device=device)
    return ids.to(device), cu, cbl, tri, meta


def _outputs(total, groups, topk, meta, device):
    rows = meta.total_blocks * groups
    cap = total * groups * topk
    # filled with a marker so that unwritten entries would show
    return (torch.full((rows + 1,), 12345, dtype=torch.int32, device=device),
            torch.full((cap,), 777, dtype=torch.int32, device=device),
            torch.full((cap,), 777, dtype=torch.int32, device=device))


def _args(ids, cu, cbl, tri, meta, groups, topk):
    total = ids.shape[0]
    counter_elems = groups * meta.tri_prefix[-1]
    return (ids.data_ptr(), cu.data_ptr(), cbl.data_ptr(), tri.data_ptr(), meta.num_seqs, total, groups, topk,
            meta.block_size, meta.total_blocks, counter_elems)


@pytest.mark.parametrize("seed", [0])
def test_noalloc_build_matches_workspace_build(seed, device):
    lib = _lib.lib()
    stream = _lib.stream_of(device)
    for lengths, groups, topk, block in (([700, 0, 1500, 333], 4, 6, 64), ([129, 40], 2, 3, 32)):
        ids, cu, cbl, tri, meta = _case(lengths, groups, topk, block, seed, device)
        total = ids.shape[0]
        args = _args(ids, cu, cbl, tri, meta, groups, topk)
        ref = _outputs(total, groups, topk, meta, device)
        ws = torch.empty(args[-1] + meta.total_blocks * groups, dtype=torch.int32, device=device)
        with torch.cuda.device(device):
            assert lib.msa_k2q_build(*args, *(x.data_ptr() for x in ref), ws.data_ptr(), stream) == 0
        got = _outputs(total, groups, topk, meta, device)
        with torch.cuda.device(device):
            assert lib.msa_k2q_build_noalloc(*args, *(x.data_ptr() for x in got), stream) == 0
        torch.cuda.synchronize()
        for a, b, what in zip(got, ref, ("row_ptr", "query_indices", "slot_indices")):
            assert torch.equal(a, b), f"{lengths}: {what} differs"
        assert int(ref[0][-1]) > 0


def test_noalloc_build_refuses_beyond_its_array(device):
    lib = _lib.lib()
    ids, cu, cbl, tri, meta = _case([100], 2, 2, 32, 1, device)
    args = list(_args(ids, cu, cbl, tri, meta, 2, 2))
    args[-1] = NOALLOC_MAX_ELEMS  # counters plus row totals no longer fit: refused before any launch
    out = _outputs(100, 2, 2, meta, device)
    with torch.cuda.device(device):
        rc = lib.msa_k2q_build_noalloc(*args, *(x.data_ptr() for x in out), _lib.stream_of(device))
    assert rc == 2
    torch.cuda.synchronize()
    assert int(out[0][0]) == 12345  # nothing was written
