"""GPU: umic_stream_read reads every byte it is given, once.

The read-ceiling helper xor-folds what each workgroup reads into one word
per workgroup.  XOR is associative and commutative, so the xor of all fold
words equals the xor of every 32-bit word of the buffer, whatever the grid
walk.  A skipped 16-byte load drops its words from the fold and a doubled
one cancels them, so either changes the fold of random data.  Sizes cover a
partial last trip of the grid, a buffer smaller than one trip, and one
16-byte load.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from umic import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("nbytes", [16, 4096, 2048 * 256 * 16 * 8 + 16 * 1000, 33_554_432])
def test_fold_equals_the_xor_of_every_word(nbytes):
    print(f"umic_stream_read bytes={nbytes}", flush=True)
    rng = np.random.default_rng(nbytes)
    words = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint64).astype(np.uint32)
    buf = torch.from_numpy(words.view(np.int32)).to(DEV)
    fold = torch.full((_lib.UMIC_STREAM_READ_GRID,), -1, dtype=torch.int32, device=DEV)
    _lib.call("umic_stream_read", buf.data_ptr(), nbytes, fold.data_ptr(), _lib.stream_of(buf))
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(fold.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(words)


def test_misaligned_and_ragged_sizes_are_rejected():
    buf = torch.zeros(64, dtype=torch.int32, device=DEV)
    fold = torch.zeros(_lib.UMIC_STREAM_READ_GRID, dtype=torch.int32, device=DEV)
    rd = _lib.lib().umic_stream_read
    st = _lib.stream_of(buf)
    assert rd(buf.data_ptr(), 20, fold.data_ptr(), st) == _lib.UMIC_ERR_UNSUPPORTED
    assert rd(buf.data_ptr() + 4, 32, fold.data_ptr(), st) == _lib.UMIC_ERR_UNSUPPORTED
    assert rd(buf.data_ptr(), 0, fold.data_ptr(), st) == _lib.UMIC_OK
