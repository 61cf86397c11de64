"""The HBM streaming probe (jl_hbm_stream in libjl_bench.so) behind bench.py's achievable
bandwidth: a copy reproduces its source, a write fills the whole range with
the probe's pattern, and a read (streaming or one word per 256-byte block)
leaves its buffers alone."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def test_stream_probe_copy_write_read():
    from bench import load_probe
    from iclr_2027_jointoom_amd._abi import check

    lib = load_probe()
    n = (1 << 20) + 4096  # not a multiple of the grid's stride
    src = torch.randint(0, 1 << 30, (n // 4,), dtype=torch.int32, device="cuda")
    dst = torch.zeros_like(src)
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    # grid-stride non-temporal and plain stores, chunked non-temporal and plain
    for copy_kind, write_kind in ((2, 1), (4, 3), (7, 6), (9, 8)):
        dst.zero_()
        check(lib.jl_hbm_stream(copy_kind, src.data_ptr(), dst.data_ptr(), n, sink.data_ptr(), 37, stream), "copy")
        torch.cuda.synchronize()
        assert torch.equal(src, dst)
        check(lib.jl_hbm_stream(write_kind, None, dst.data_ptr(), n, sink.data_ptr(), 37, stream), "write")
        torch.cuda.synchronize()
        words = dst.view(-1, 4).cpu().numpy().view(np.uint32)
        assert (words[:, 0] == 0x01010101).all() and (words[:, 1] == 0x02020202).all()
        assert (words[:, 2] == 0x03030303).all() and (words[:, 3] < 37).all()
    before = src.clone()
    # kind 10: one 16-byte read per 256-byte block (the fetch-granularity probe)
    for read_kind in (0, 5, 10):
        check(lib.jl_hbm_stream(read_kind, src.data_ptr(), None, n, sink.data_ptr(), 37, stream), "read")
        torch.cuda.synchronize()
        assert torch.equal(src, before)
    assert lib.jl_hbm_stream(11, src.data_ptr(), dst.data_ptr(), n, sink.data_ptr(), 37, stream) == -1
    assert lib.jl_hbm_stream(10, src.data_ptr(), None, n - 16, sink.data_ptr(), 37, stream) == -1
    assert lib.jl_hbm_stream(2, src.data_ptr(), dst.data_ptr(), n + 8, sink.data_ptr(), 37, stream) == -1
