"""The measurement probes behind the bench's measured peaks and decode
floor (rlxq_peak_probe): each read probe reads every byte of its buffer
exactly once (the XOR of the per-workgroup sink words equals the XOR of the
buffer's dwords), the counts they return are the work they issue, and bad
arguments are refused before any launch."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [4096, 10485760, 62914560 + 4096])
@pytest.mark.parametrize("kind", ["READ", "READ4"])
def test_read_probes_read_every_byte_once(ctx, kind, nbytes):
    import torch
    import rlxq

    g = torch.Generator(device="cuda")
    g.manual_seed(nbytes)
    buf = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), device="cuda", dtype=torch.int32, generator=g)
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    k = rlxq.PROBE_READ if kind == "READ" else rlxq.PROBE_READ4
    assert ctx.peak_probe(k, nbytes, buf=buf, sink=sink) == nbytes
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(buf.cpu().numpy().view(np.uint32))
    assert got == want


@pytest.mark.parametrize("nbytes", [81920, 62914560])
def test_tile20_probe_reads_every_block_once(ctx, nbytes):
    """The batched-decode lane-pattern probe (rows of 2560 bytes, one 20-byte
    block per lane): every dword of every block read exactly once."""
    import torch
    import rlxq

    g = torch.Generator(device="cuda")
    g.manual_seed(nbytes + 1)
    buf = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), device="cuda", dtype=torch.int32, generator=g)
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    assert ctx.peak_probe(rlxq.PROBE_TILE20, nbytes, buf=buf, sink=sink) == nbytes
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(buf.cpu().numpy().view(np.uint32))
    assert got == want


def test_probe_counts_and_refusals(ctx):
    import torch
    import rlxq

    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert ctx.peak_probe(rlxq.PROBE_MFMA, 3, sink=sink) == cus * 8 * 4 * 3 * 4 * 32768
    buf = torch.zeros(2048, dtype=torch.int32, device="cuda")
    for kind in (rlxq.PROBE_READ, rlxq.PROBE_READ4):
        with pytest.raises(rlxq.RlxqError) as e:
            ctx.peak_probe(kind, 4000, buf=buf, sink=sink)
        assert e.value.status == rlxq.E_ALIGN
        with pytest.raises(rlxq.RlxqError) as e:
            ctx.peak_probe(kind, 4096, buf=None, sink=sink)
        assert e.value.status == rlxq.E_NULL
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.peak_probe(rlxq.PROBE_READ4, (1 << 30) + 4096, buf=buf, sink=sink)
    assert e.value.status == rlxq.E_SHAPE
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.peak_probe(rlxq.PROBE_TILE20, 81920 + 4096, buf=buf, sink=sink)
    assert e.value.status == rlxq.E_ALIGN
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.peak_probe(rlxq.PROBE_TILE20, 65537 * 81920, buf=buf, sink=sink)
    assert e.value.status == rlxq.E_SHAPE
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.peak_probe(7, 4096, buf=buf, sink=sink)
    assert e.value.status == rlxq.E_SHAPE
    torch.cuda.synchronize()
