"""GPU parity of jf_tree_gather (through the C ABI) against the oracle and
the closed form: bit-exact data after the in-place gather, for the 16-byte
path (contiguous rows of 8-column runs) and the element path (strided
columns), and the arguments it must reject."""
import numpy as np
import pytest

import jf_sampler as J
import oracle as O
from gather_cases import gather_case, gather_closed_form

pytestmark = pytest.mark.gpu


def run_gpu(data, path, retained, p):
    import torch
    dev = torch.device("cuda", 0)
    d = torch.from_numpy(data.view(np.int16)).to(dev)
    pr = torch.from_numpy(path.view(np.int32)).to(dev)
    rt = torch.from_numpy(retained.view(np.int32)).to(dev)
    J.tree_gather(J.tree_gather_args(d, pr, rt, **p))
    torch.cuda.synchronize()
    return d.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("shape", [
    dict(columns=4096, inner=4096, pad=0),                                   # 16-byte path
    dict(columns=1024, inner=128, inner_stride=1, outer_stride=128, pad=8),  # 16-byte, grouped
    dict(columns=40, inner=40, pad=3),                                       # element path
    dict(columns=48, inner=8, inner_stride=2, outer_stride=20),
    dict(columns=30, inner=5, inner_stride=1, outer_stride=7)])
def test_tree_gather_matches_oracle(shape):
    rng = np.random.default_rng(sum(shape.values()))
    data, path, retained, p = gather_case(rng, lanes=6, layers=4, **shape)
    print(f"gather case {p}", flush=True)
    got = run_gpu(data, path, retained, p)
    want = O.tree_gather(data, path, retained, **p)
    assert np.array_equal(got, want)
    if p["columns"] <= 64:
        assert np.array_equal(got, gather_closed_form(data, path, retained, p))


def test_tree_gather_rejects_bad_extent():
    import torch
    dev = torch.device("cuda", 0)
    d = torch.zeros(100, dtype=torch.int16, device=dev)
    pr = torch.zeros(8, dtype=torch.int32, device=dev)
    rt = torch.zeros(1, dtype=torch.int32, device=dev)
    a = J.tree_gather_args(d, pr, rt, columns=10, inner=10, inner_stride=1, outer_stride=10,
                           row_stride=10, lane_stride=160, layer_stride=160, layers=1, lanes=1,
                           rows=16)
    with pytest.raises(J.JfError):
        J.tree_gather(a)
