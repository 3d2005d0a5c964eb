"""qlinear_stream_read (the single-kernel HBM read floor the skinny-M kernels are compared with):
every 16-byte chunk is read exactly once -- the xor of the per-workgroup words equals the xor of
all the buffer's 32-bit words -- for sizes with and without a partial last round of loads."""
import numpy as np
import pytest
import torch

from comfy_ui_gfx906_tools_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096, 1 << 20, (1 << 20) + 48, 26_214_400 + 5_242_880])
def test_stream_read_reads_every_chunk_once(nbytes):
    g = np.random.default_rng(nbytes)
    host = g.integers(0, 2**32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    buf = torch.from_numpy(host.view(np.int32)).cuda()
    out = _lib.stream_read(buf)
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host)


def test_stream_read_argument_checks():
    lib = _lib.load_library()
    buf = torch.zeros(64, dtype=torch.uint8, device="cuda")
    out = torch.zeros(1024, dtype=torch.int32, device="cuda")
    assert lib.qlinear_stream_read(buf.data_ptr(), 24, out.data_ptr(), None) != 0
    assert "multiple of 16" in lib.qlinear_last_error().decode()
    assert lib.qlinear_stream_read(buf.data_ptr() + 8, 32, out.data_ptr(), None) != 0
