"""The streaming-read probe (mle_probe_stream_read), a measurement aid the benchmark
sets each decode Linear against: it reads buffers of any multiple of 16 bytes (sizes
below one grid stride, ragged tails, the benchmark's weight sizes) without error,
writes nothing (the sink keeps its value for buffers whose words never fold to the
probe's constant), and rejects a size that is not a multiple of 16."""
import pytest

from helpers import note
from llmengine_amd import capi

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [0, 16, 4096 * 256 * 16 - 16, 4096 * 256 * 16 * 3 + 48,
                                    47_906_816])
def test_probe_reads_without_writing(dev, nbytes):
    import torch
    note(f"stream-read probe {nbytes} bytes")
    src = torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=dev)
    sink = torch.full((4,), 7, dtype=torch.int32, device=dev)
    capi.probe_stream_read(src, nbytes, sink)
    torch.cuda.synchronize()
    assert sink.cpu().tolist() == [7, 7, 7, 7]


def test_probe_rejects_ragged_size(dev):
    import torch
    src = torch.zeros(64, dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    code, msg = capi.probe_stream_read_status(src, 40, sink)
    assert code == 1 and "multiple of 16" in msg
