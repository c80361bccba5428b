"""GPU: the stream handle the wrappers pass to the C ABI, and the benchmark's device-side hold.

testt_amd._ext.stream_of uses torch's raw current-stream query (not public API) and falls back
to torch.cuda.current_stream().cuda_stream; both must name the same stream, on the default
stream and inside a stream context.  soupk_bench_hold must keep its stream busy for about the
time asked (the benchmark queues its timed launches behind it) and then end."""

import pytest
import torch

from testt_amd import _ext

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def test_raw_and_public_stream_queries_agree():
    t = torch.empty(1, device=DEV)
    assert _ext.stream_of(t) == _ext.public_stream_of(t)
    side = torch.cuda.Stream(DEV)
    with torch.cuda.stream(side):
        assert _ext.stream_of(t) == _ext.public_stream_of(t) == side.cuda_stream
    assert _ext.stream_of(t) == torch.cuda.current_stream(DEV).cuda_stream


def test_bench_hold_waits_then_ends():
    lib = _ext.lib()
    s = torch.cuda.current_stream(DEV)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    assert lib.soupk_bench_hold(0.0, s.cuda_stream) == 0    # (first launch loads the code)
    for us in (0.0, 500.0, 5000.0):
        torch.cuda.synchronize(DEV)
        e0.record(s)
        assert lib.soupk_bench_hold(us, s.cuda_stream) == 0
        e1.record(s)
        torch.cuda.synchronize(DEV)
        got = e0.elapsed_time(e1) * 1e3
        print(f"hold {us} us -> {got:.1f} us", flush=True)
        assert us * 0.95 <= got <= us * 1.2 + 200.0
