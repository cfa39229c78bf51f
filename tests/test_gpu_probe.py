"""The ceiling probes bench.py measures its ceilings with: the streaming copy
reproduces its source exactly (whole passes and a ragged tail), the
streaming read runs and leaves its inputs untouched, and the MFMA probe runs
every operand pairing, leaves its operands untouched and refuses what it
cannot run."""
import pytest
import torch

import hxm
from hxm._lib import lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 48, 64 << 20])
def test_probe_copy_reproduces_its_source(dev, nbytes):
    print(f"probe_copy {nbytes} bytes", flush=True)
    g = torch.Generator().manual_seed(nbytes % 1000)
    src = torch.randint(0, 256, (nbytes,), generator=g, dtype=torch.uint8).to(dev)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device=dev)
    hxm.check(lib.hxm_probe_copy(src.data_ptr(), dst.data_ptr(), nbytes,
                                 torch.cuda.current_stream().cuda_stream), "hxm_probe_copy")
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert int(dst[nbytes:].sum()) == 0


def test_probe_read_runs_and_writes_at_most_the_sink(dev):
    nbytes = (45 << 20) + 16 * 7
    print(f"probe_read {nbytes} bytes", flush=True)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev)
    keep = src.clone()
    sink = torch.zeros(8192, dtype=torch.int32, device=dev)
    hxm.check(lib.hxm_probe_read(src.data_ptr(), nbytes, sink.data_ptr(),
                                 torch.cuda.current_stream().cuda_stream), "hxm_probe_read")
    torch.cuda.synchronize()
    assert torch.equal(src, keep)


@pytest.mark.parametrize("a_dt,b_dt", [(hxm.I8, hxm.I8), (hxm.F16, hxm.F16), (hxm.BF16, hxm.BF16),
                                       (hxm.F16, hxm.I8)])
def test_probe_mfma_runs_and_leaves_its_operands(dev, a_dt, b_dt):
    """The MFMA ceiling probe runs every operand pairing on a small grid,
    reads its operands without changing them, and writes the sink at most
    where the fold equals the rare value; wrapped windows (operands smaller
    than a wave's 8 KiB) stay inside the buffers."""
    print(f"probe_mfma {a_dt} x {b_dt}", flush=True)
    g = torch.Generator().manual_seed(a_dt * 10 + b_dt)
    a = torch.randint(-127, 128, (64 << 10,), generator=g, dtype=torch.int8).to(dev)
    b = torch.randint(-127, 128, (4096 + 48,), generator=g, dtype=torch.int8).to(dev)
    ka, kb = a.clone(), b.clone()
    sink = torch.zeros(8192, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    hxm.check(lib.hxm_probe_mfma(a.data_ptr(), a.numel(), b.data_ptr(), b.numel(), a_dt, b_dt,
                                 64, 16, sink.data_ptr(), st), "hxm_probe_mfma")
    torch.cuda.synchronize()
    assert torch.equal(a, ka) and torch.equal(b, kb)
    assert int((sink[16:] != 0).sum()) == 0


def test_probe_mfma_refusals(dev):
    a = torch.zeros(8192, dtype=torch.int8, device=dev)
    sink = torch.zeros(8192, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    p, s = a.data_ptr(), sink.data_ptr()
    assert lib.hxm_probe_mfma(p, 8192, p, 8192, hxm.I8, hxm.F16, 32, 1, s, st) != 0
    assert "unsupported-dtype" in hxm.last_error()
    assert lib.hxm_probe_mfma(p, 8192, p, 8192, hxm.I8, hxm.I8, 48, 1, s, st) != 0
    assert lib.hxm_probe_mfma(p, 8000 + 8, p, 8192, hxm.I8, hxm.I8, 32, 1, s, st) != 0
    assert lib.hxm_probe_mfma(p, 8192, p, 8192, hxm.I8, hxm.I8, 32, 0, s, st) != 0
    assert lib.hxm_probe_mfma(p, 8192, p, 8192, hxm.I8, hxm.I8, 32, 1, None, st) != 0
    # past 2^24 MFMAs per wave a launch would hold the device for seconds
    assert lib.hxm_probe_mfma(p, 8192, p, 8192, hxm.I8, hxm.I8, (1 << 24) + 32, 1, s,
                              st) != 0
    assert "2^24" in hxm.last_error()
