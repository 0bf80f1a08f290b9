"""air_hip_stream_read: the streaming-floor pass the benchmark prices each
M = 1 linear against.  Its checksum is the XOR of the buffer's 32-bit words
(numpy computes the same), whatever the size relative to its chunks."""
import numpy as np
import pytest

from air_amd import capi


@pytest.mark.gpu
@pytest.mark.parametrize("nbytes,sink_words", [(16, 1), (1024, 4), (8192 + 48, 4096), (57344 * 3 + 16, 2),
                                               (13_647_872, 65536), (72_138_752, 300), (72_138_752, 1)])
def test_stream_read_checksum(torch_cuda, hip_ctx, nbytes, sink_words):
    torch = torch_cuda
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    data = torch.from_numpy(host.view(np.int32)).to("cuda:0")
    sink = torch.zeros(sink_words, dtype=torch.int32, device="cuda:0")
    hip_ctx.stream_read(data, nbytes, sink, sink_words)
    torch.cuda.synchronize()
    want = np.bitwise_xor.reduce(host) if host.size else np.uint32(0)
    assert int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))) == int(want)


@pytest.mark.gpu
def test_stream_read_refuses_ragged_sizes(torch_cuda, hip_ctx):
    torch = torch_cuda
    data = torch.zeros(64, dtype=torch.int32, device="cuda:0")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda:0")
    with pytest.raises(capi.HipError):
        hip_ctx.stream_read(data, 20, sink, 4)
    with pytest.raises(capi.HipError):
        hip_ctx.stream_read(data, 16, sink, 0)
