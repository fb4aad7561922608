"""The measurement probes beside the decode kernels run through the C-ABI:
the LDS read-pattern probe gives positive cycle counts with the same-bank
pattern well above the contiguous one, and a gather-probe variant reads a
small cache (its sink stays untouched unless a checksum collides)."""
import ctypes

import pytest
import torch

from amd_optimization_challenge_amd import _lib, ops

pytestmark = pytest.mark.gpu


def test_lds_probe_patterns(cuda):
    print("lds probe: 5 patterns, 8 groups", flush=True)
    lib = _lib.load()
    cyc = torch.zeros(4 * 8, dtype=torch.float32, device=cuda)
    sink = torch.zeros(256, dtype=torch.int32, device=cuda)
    per = []
    for pat in range(5):
        _lib.check(lib.mla_probe_lds(pat, 256, 8, ctypes.c_void_p(cyc.data_ptr()), ctypes.c_void_p(sink.data_ptr()),
                                     ops._stream()), "mla_probe_lds")
        torch.cuda.synchronize()
        assert bool((cyc > 0).all()), pat
        per.append(float(cyc.mean()))
    assert per[4] > 2 * per[0], per
    with pytest.raises(_lib.MlaLibraryError):
        _lib.check(lib.mla_probe_lds(5, 1, 1, ctypes.c_void_p(cyc.data_ptr()), ctypes.c_void_p(sink.data_ptr()),
                                     ops._stream()), "mla_probe_lds")


def test_gather_probe_variant_runs(cuda):
    print("gather probe: fp8 rows, 4 waves, 4 stages", flush=True)
    g = torch.Generator(device=cuda).manual_seed(5)
    rows = torch.randint(0, 256, (4096, 576), dtype=torch.uint8, device=cuda, generator=g)
    idx = torch.randperm(4096, device=cuda, generator=g).to(torch.int32)
    sink = torch.zeros(1024, dtype=torch.uint8, device=cuda)
    _lib.check(_lib.load().mla_probe_gather(0, 0, 4, 4, 16, ops._ptr(rows), 576, ops._ptr(None), 0, ops._ptr(None), 0,
                                            ops._ptr(idx), 4096, ops._ptr(sink), ops._stream()), "mla_probe_gather")
    torch.cuda.synchronize()
