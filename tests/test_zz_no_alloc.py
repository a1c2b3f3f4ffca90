"""okf_argmax_rows_noalloc (the entry point that allocates nothing) against
okf_argmax_rows through the C ABI: two calls in a row, the second smaller,
and a call past the fixed scratch refused.  Bit-exact indices."""
import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")
import chatokf_amd as ok  # noqa: E402

pytestmark = pytest.mark.gpu


def test_argmax_noalloc_matches_argmax_rows():
    enc = ok.Enc(0)
    try:
        rng = np.random.default_rng(2024)
        for n, rows in ((248320, 5), (70001, 2)):  # second call smaller
            x = rng.standard_normal((rows, n)).astype(np.float32)
            x[0, n // 2] = x[0, n - 1] = 50.0  # a tie: the lower index wins
            xd = torch.from_numpy(x).cuda()
            a = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
            b = torch.full((rows,), -9, dtype=torch.int32, device="cuda")
            enc.argmax_rows_noalloc(xd, n, rows, a)
            enc.argmax_rows(xd, n, rows, b)
            enc.sync()
            ga, gb = a.cpu().numpy(), b.cpu().numpy()
            assert np.array_equal(ga, gb)
            assert np.array_equal(ga, oracle.argmax_rows(x))
        # beyond the fixed scratch: rows * ceil(n / 1024) > 131072 pairs, or
        # rows > 4096 (refused before anything is read, so a small buffer does)
        buf = torch.zeros(16, device="cuda")
        out = torch.empty(16, dtype=torch.int32, device="cuda")
        for n, rows in ((33 * 1024, 4096), (1, 4097)):
            with pytest.raises(ok.OkfError) as e:
                enc.argmax_rows_noalloc(buf, n, rows, out)
            assert e.value.status == ok.OKF_E_SHAPE
    finally:
        enc.close()
