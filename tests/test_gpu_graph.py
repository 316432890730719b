"""jf_sample_static under HIP graph capture: three selections of the headline
workload (C2, 64 rows, penalties) captured into one graph through torch's
capture of the current stream, then replayed four times with the program's
own eager work (jf_sample) and a synchronization between replays; every
replay's tokens equal the eager selections'. The static entry point passes
its row parameters as kernel arguments and clears its counters with a fill
kernel, so a replay needs nothing from the host."""
import numpy as np
import pytest

import bench
import jf_sampler as J

pytestmark = pytest.mark.gpu


def test_static_entry_point_replays_under_a_hip_graph():
    import torch
    w = bench.build_workload(2, "auto")
    g = bench.GpuStep(w)
    V, rows, n = w["V"], w["rows"], 3
    want = []
    for i in range(n):
        g.out.fill_(-1)
        g.step(i)
        torch.cuda.synchronize()
        want.append(g.out.cpu().numpy().copy())
    outs = [torch.full((rows,), -1, dtype=torch.int32, device="cuda") for _ in range(n)]
    args = []
    for i in range(n):
        a = J.JfSampleArgs.from_buffer_copy(g.kw[i][0])
        a.out_tokens = outs[i].data_ptr()
        args.append(a)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for a in args:  # outside capture: the scratch address lookup happens here
            J.sample_static(V, a)
    torch.cuda.synchronize()
    for i in range(n):
        np.testing.assert_array_equal(outs[i].cpu().numpy(), want[i])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for a in args:
            J.sample_static(V, a)
    for rep in range(4):
        for o in outs:
            o.fill_(-1)
        g.step(rep + 5)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i in range(n):
            np.testing.assert_array_equal(outs[i].cpu().numpy(), want[i])
    del graph
