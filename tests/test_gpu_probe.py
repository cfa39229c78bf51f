"""The HBM probes bench.py measures its ceilings with: the streaming copy
reproduces its source exactly (whole passes and a ragged tail), and the
streaming read runs and leaves its inputs untouched."""
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
