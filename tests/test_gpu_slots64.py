"""A standard build whose graph has more than 2^32 forward slots (N * R), so
the reverse CSR is sorted in parts (k_rev_keys over source ranges, then
k_wide_offsets / k_wide_gather). At this size only invariants can be
checked; the split path itself is compared bit for bit with the oracle at
small sizes in test_gpu_parity.py (DANCE_REVERSE_PART_ITEMS)."""
import pytest

import dance_amd as D

pytestmark = pytest.mark.gpu


def test_build_beyond_2_pow_32_slots():
    import torch
    N, dim, R, L, C, steps = (1 << 26) + 4096, 8, 64, 64, 64, 32
    assert N * R > 0xFFFFFFFF
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(11)
    x = torch.randint(0, 256, (N, dim), dtype=torch.uint8, device=dev, generator=gen)
    graph = torch.empty((N, R), dtype=torch.int32, device=dev)
    degree = torch.empty(N, dtype=torch.int32, device=dev)
    D.vamana_build_resident(x.data_ptr(), D.DTYPE_U8, N, dim, R, L, C, steps, graph.data_ptr(), degree.data_ptr())
    torch.cuda.synchronize()
    del x
    d = degree.long()
    assert int(d.min()) >= 1 and int(d.max()) <= R
    invalid = selfl = dup = pad = cross = 0
    half = N // 2
    col = torch.arange(R, device=dev)[None, :]
    for b in range(0, N, 1 << 22):
        e = min(N, b + (1 << 22))
        g = graph[b:e].long() & 0xFFFFFFFF
        live = col < d[b:e, None]
        rows = torch.arange(b, e, device=dev)[:, None]
        invalid += int((live & (g >= N)).sum())
        selfl += int((live & (g == rows)).sum())
        pad += int((~live & (g != 0xFFFFFFFF)).sum())
        srt = torch.sort(torch.where(live, g, (-col - 1).expand_as(g)), dim=1).values
        dup += int((srt[:, 1:] == srt[:, :-1]).sum())
        # edges whose source and target lie on different sides of the middle
        cross += int((live & ((rows < half) != (g < half))).sum())
    assert invalid == 0 and selfl == 0 and dup == 0 and pad == 0
    assert cross > 0
    assert D.last_kernel_profile()["reverse_edges"] > 0
