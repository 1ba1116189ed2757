"""GPU: umic_stream_read reads every byte it is given, once; umic_stream_copy
copies every byte it is given and nothing past them.

The read-ceiling helper xor-folds what each workgroup reads into one word
per workgroup.  XOR is associative and commutative, so the xor of all fold
words equals the xor of every 32-bit word of the buffer, whatever the grid
walk.  A skipped 16-byte load drops its words from the fold and a doubled
one cancels them, so either changes the fold of random data.  Sizes cover a
partial last trip of the grid, a buffer smaller than one trip, and one
16-byte load.  The copy's destination carries a guard band of a known
pattern past its end that must survive; its sizes cover a partial last
workgroup (512 16-byte loads each), a partial last lane pair, one load, and
a BASELINE-sized side.
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


@pytest.mark.parametrize("nbytes", [16, 512 * 16 * 3 + 16 * 257, 512 * 16 * 5 + 16, 25_399_296])
def test_copy_is_exact_and_stays_in_its_range(nbytes):
    print(f"umic_stream_copy bytes={nbytes}", flush=True)
    guard = 4096
    g = torch.Generator(device="cpu").manual_seed(nbytes)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=g).to(DEV)
    dst = torch.full((nbytes + guard,), 0xA5, dtype=torch.uint8, device=DEV)
    _lib.call("umic_stream_copy", src.data_ptr(), dst.data_ptr(), nbytes, _lib.stream_of(src))
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert bool((dst[nbytes:] == 0xA5).all())


def test_copy_rejections():
    buf = torch.zeros(1024, dtype=torch.int32, device=DEV)
    cp = _lib.lib().umic_stream_copy
    st = _lib.stream_of(buf)
    p = buf.data_ptr()
    assert cp(p, p + 2048, 1000, st) == _lib.UMIC_ERR_UNSUPPORTED
    assert cp(p, p + 2052, 1024, st) == _lib.UMIC_ERR_UNSUPPORTED
    assert cp(p, p + 1024, 2048, st) == _lib.UMIC_ERR_INVALID_ARG
    assert cp(p, p + 2048, 0, st) == _lib.UMIC_OK
