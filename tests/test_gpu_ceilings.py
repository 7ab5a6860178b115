"""GPU checks of the measured-ceiling kernels the benchmark's roofline uses
(prism_amd/csrc/peak.hip): the tile stream copies the tiles it claims into
LDS, and the HBM copy copies."""
import ctypes

import numpy as np
import pytest
import torch

from tests.test_gpu_parity import say

pytestmark = pytest.mark.gpu

M64 = (1 << 64) - 1


def _lcg(h):
    return (h * 6364136223846793005 + 1442695040888963407) & M64


@pytest.mark.parametrize("ntiles,steps", [(1, 1), (7, 2), (11520, 3)])
def test_tile_stream_peak_copies_its_tiles(ntiles, steps):
    """Each workgroup's last stage holds tile ta of its last step at LDS offset
    0 (lane 0 of instruction 0 reads the tile's first 16 bytes): the sink word
    equals the source word at ta * 16384 bytes.  ta follows the kernel's
    per-workgroup LCG (h0 = block + 1; two draws per step, (h >> 17) mod
    ntiles)."""
    from prism_amd import _lib
    say("tile stream", ntiles, steps)
    words = ntiles * 16384 // 4
    src = torch.arange(words, device="cuda", dtype=torch.int32)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.full((2 * cus,), -1, device="cuda", dtype=torch.int32)
    moved = ctypes.c_int64(0)
    _lib.call("prism_tile_stream_peak", src.data_ptr(), ntiles * 16384, steps, sink.data_ptr(), sink.numel(),
              ctypes.addressof(moved), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert moved.value == 2 * cus * steps * 2 * 16384
    want = []
    for b in range(2 * cus):
        h = b + 1
        for _ in range(steps):
            h = _lcg(h)
            ta = (h >> 17) % ntiles
            h = _lcg(h)
        want.append(ta * 4096)
    assert np.array_equal(sink.cpu().numpy(), np.array(want, np.int64).astype(np.int32))


def test_tile_stream_peak_rejects_bad_sizes():
    from prism_amd import _lib
    src = torch.zeros(4096, device="cuda", dtype=torch.int32)
    sink = torch.zeros(4096, device="cuda", dtype=torch.int32)
    moved = ctypes.c_int64(0)
    s = torch.cuda.current_stream().cuda_stream
    with pytest.raises(Exception):  # not a whole number of 16 KB tiles
        _lib.call("prism_tile_stream_peak", src.data_ptr(), 10000, 1, sink.data_ptr(), sink.numel(),
                  ctypes.addressof(moved), s)
    with pytest.raises(Exception):  # sink too short for 2 x CUs workgroups
        _lib.call("prism_tile_stream_peak", src.data_ptr(), 16384, 1, sink.data_ptr(), 1, ctypes.addressof(moved), s)


def test_copy_peak_copies():
    from prism_amd import _lib
    n = 1 << 20
    src = torch.arange(n, device="cuda", dtype=torch.int32)
    dst = torch.zeros_like(src)
    _lib.call("prism_copy_peak", src.data_ptr(), dst.data_ptr(), 4 * n, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
