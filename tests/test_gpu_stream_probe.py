"""glm53_stream_probe (the bandwidth ceilings bench.py reports) through the
C ABI: the non-temporal copy reproduces its source byte for byte, also for a
size that leaves a partial pass of the grid-stride loop, and the two read
forms run to completion without touching their 16-byte sink."""
import pytest
import torch

from conftest import log_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096 + 16, (8 << 20) + 48])
def test_stream_probe_copy_exact_and_reads_complete(cuda, nbytes):
    import _glm53_lib as lib
    L = lib.load()
    stream = lib.stream_handle(cuda)
    g = torch.Generator(device=cuda).manual_seed(nbytes)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=cuda, generator=g)
    dst = torch.zeros(nbytes + 32, dtype=torch.uint8, device=cuda)
    log_case("stream probe", f"{nbytes} bytes")
    lib.check(L.glm53_stream_probe(2, src.data_ptr(), dst.data_ptr(), nbytes, stream), "glm53_stream_probe copy")
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert int(dst[nbytes:].count_nonzero()) == 0          # nothing past the end
    sink = torch.zeros(16, dtype=torch.uint8, device=cuda)
    for kind in (0, 1):
        lib.check(L.glm53_stream_probe(kind, src.data_ptr(), sink.data_ptr(), nbytes, stream), "glm53_stream_probe read")
    torch.cuda.synchronize()
    assert int(sink.count_nonzero()) == 0   # written only for one magic fold value of the data
