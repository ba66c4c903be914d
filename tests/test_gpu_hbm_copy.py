"""hh_hbm_copy, the streaming copy the measurements are calibrated with:
byte-exact for every alignment of source and destination, head / tail
lengths around the 16-byte chunks, and overlap refused."""
import numpy as np
import pytest

import gpu_util as G

pytestmark = pytest.mark.gpu


def test_copy_alignments_and_lengths():
    import haagenti_amd as H
    T = G.torch()
    rng = np.random.default_rng(31)
    src = T.from_numpy(rng.integers(0, 256, 1 << 20, dtype=np.uint8)).cuda()
    for so, do, n in [(0, 0, 1 << 20), (0, 0, 16), (3, 3, 1000), (5, 9, 777), (1, 0, 65537),
                      (15, 15, 17), (0, 0, 0), (7, 7, 1), (0, 0, (1 << 20) - 64)]:
        dst = T.full(((1 << 20) + 64,), 0xA5, dtype=T.uint8, device="cuda")
        G.ctx().hbm_copy(dst[do:], src[so:], n, stream=G.stream())
        G.sync()
        d = dst.cpu().numpy()
        assert (d[do:do + n] == src[so:so + n].cpu().numpy()).all(), (so, do, n)
        assert (d[:do] == 0xA5).all() and (d[do + n:] == 0xA5).all(), (so, do, n)


def test_overlap_refused():
    import haagenti_amd as H
    T = G.torch()
    a = T.zeros(4096, dtype=T.uint8, device="cuda")
    with pytest.raises(H.HaagentiError) as e:
        G.ctx().hbm_copy(a[100:], a, 1000)
    assert e.value.code == H.INVALID_ARGUMENT
