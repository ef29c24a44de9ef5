"""GPU: the HBM stream probes bench.py reads the primitives against
(mg_probe_stream, a measurement aid with no reference counterpart) move
exactly the data they claim to."""
import pytest

import mgprims as M

pytestmark = pytest.mark.gpu


def test_copy_write_2r2w(prims):
    import torch
    g = torch.Generator(device="cuda:0")
    g.manual_seed(5)
    n = (1 << 20) + 256  # not a multiple of the 4096-byte work-group span
    a = torch.randint(0, 2 ** 31 - 1, (n,), generator=g, device="cuda:0", dtype=torch.int32)
    b = torch.zeros_like(a)
    prims.probe_stream(M.Prims.PROBE_COPY, a, b)
    assert torch.equal(a, b)

    prims.probe_stream(M.Prims.PROBE_WRITE, None, b)
    i = torch.arange(n // 4, device="cuda:0", dtype=torch.int32)
    want = torch.stack([i, torch.ones_like(i), torch.full_like(i, 2), torch.full_like(i, 3)], 1).reshape(-1)
    assert torch.equal(b, want)

    c = torch.randint(0, 2 ** 31 - 1, (n,), generator=g, device="cuda:0", dtype=torch.int32)
    d = torch.zeros_like(a)
    a0 = a.clone()
    prims.probe_stream(M.Prims.PROBE_2R2W, a, None, c, d)
    s = (a0.to(torch.int64) + c.to(torch.int64)) & 0xFFFFFFFF
    s = torch.where(s >= 2 ** 31, s - 2 ** 32, s).to(torch.int32)
    assert torch.equal(a, s)
    assert torch.equal(d, s ^ c)

    sink = torch.zeros(4, dtype=torch.int32, device="cuda:0")
    prims.probe_stream(M.Prims.PROBE_READ, torch.zeros(n, dtype=torch.int32, device="cuda:0"), sink)
    assert int(sink.abs().sum()) == 0


@pytest.mark.parametrize("kind", (M.Prims.PROBE_COPY_CACHED, M.Prims.PROBE_COPY_4VEC, M.Prims.PROBE_COPY_PERSISTENT))
@pytest.mark.parametrize("n", (64, (1 << 20) + 256, (9 << 20) + 4))
def test_other_copy_forms(prims, kind, n):
    """the cached, four-words-a-thread and persistent copies move every word:
    sizes below one work-group's span, past a whole number of spans, and above
    the persistent grid's 2048 groups x 256 words (so its loop runs twice)"""
    import torch
    g = torch.Generator(device="cuda:0")
    g.manual_seed(6)
    a = torch.randint(0, 2 ** 31 - 1, (n,), generator=g, device="cuda:0", dtype=torch.int32)
    b = torch.zeros(n + 8, dtype=torch.int32, device="cuda:0")
    prims.probe_stream(kind, a, b)
    assert torch.equal(b[:n], a)
    assert int(b[n:].abs().sum()) == 0  # nothing past the moved size


def test_errors(prims):
    import torch
    a = torch.zeros(64, dtype=torch.int32, device="cuda:0")
    with pytest.raises(M.MgError, match="kind"):
        prims.probe_stream(7, a, a)
    with pytest.raises(M.MgError, match="multiple of 16"):
        prims.probe_stream(M.Prims.PROBE_COPY, a[:3], a[4:7])
    with pytest.raises(M.MgError, match="misaligned"):
        prims.probe_stream(M.Prims.PROBE_COPY, a[1:5], a[8:12])
