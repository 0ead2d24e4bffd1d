"""``fd_hbm_copy``, the copy bench.py measures as the on-box HBM ceiling: the copy is exact."""
from __future__ import annotations

import pytest
import torch

from helpers import announce

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", range(6))
@pytest.mark.parametrize("nbytes", [16, 4096, 16 * 1023, 16 * 1025 * 7, 64 << 20])
def test_copy_is_exact(nbytes, shape):
    from fastdecisions_amd.hbm_copy import SHAPES, hbm_copy
    announce(f"fd_hbm_copy {nbytes} bytes, shape {SHAPES[shape]}")
    g = torch.Generator().manual_seed(nbytes % 1000)
    src = torch.randint(0, 256, (nbytes,), generator=g, dtype=torch.uint8).cuda()
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device="cuda")
    hbm_copy(src, dst[:nbytes], *SHAPES[shape])
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert not dst[nbytes:].any()  # nothing written past the end
