"""GPU check of the allocation-free decode attention (ns_decode_attention_noalloc) through the C
ABI: its output equals ns_decode_attention's, with a caller-allocated workspace, bit for bit, on
calls in a row on one GPU -- the largest size its 4 MiB scratch admits, then smaller ones, so
each call runs over what the previous call left in the scratch -- and is within the float64
oracle's tolerance."""
import pytest
import torch

from nanoserve_amd import Kernels
from oracle import decode_ref as R

pytestmark = pytest.mark.gpu

DEV = "cuda"
D = 128


@pytest.fixture(scope="module")
def k():
    return Kernels()


def rnd(*shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(torch.bfloat16).to(DEV)


def test_noalloc_matches_workspace_attention_on_calls_in_a_row(k):
    # (Hq, Hk, max_len, rows): the scratch limit (288 splits of 128 rows at Hq = 28), then
    # smaller calls: fewer splits, fewer heads, a single split
    cases = [(28, 4, 36864, 36864), (28, 4, 1024, 700), (7, 1, 300, 130), (4, 4, 64, 40)]
    for i, (Hq, Hk, max_len, n) in enumerate(cases):
        print(f"noalloc attention call {i}: Hq={Hq} Hk={Hk} max_len={max_len} rows={n}", flush=True)
        q = rnd(Hq * D, seed=20 + i)
        kc, vc = rnd(Hk, max_len, D, seed=30 + i), rnd(Hk, max_len, D, seed=40 + i)
        pos = torch.tensor([n - 1], dtype=torch.int32, device=DEV)
        work = k.decode_attention_workspace(Hq, Hk, D, max_len)
        ref = k.decode_attention(q, kc, vc, pos, Hq, Hk, D, work)
        out = torch.empty_like(ref)
        k.decode_attention_noalloc(q, kc, vc, pos, Hq, Hk, D, out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"call {i}: differs from the workspace version"
        exp = R.decode_attention(q, kc, vc, n, Hq, Hk)
        err = (out.reshape(-1).double().cpu() - exp.reshape(-1)).abs()
        assert bool((err <= 2 ** -8 * exp.reshape(-1).abs() + 1e-5).all()), f"call {i}: vs oracle"
        del kc, vc, work


def test_noalloc_rejects_beyond_its_scratch(k):
    Hq, Hk, max_len = 28, 4, 36865
    q = rnd(Hq * D, seed=1)
    kc = torch.zeros(Hk, 8, D, dtype=torch.bfloat16, device=DEV)
    pos = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.empty(1, Hq * D, dtype=torch.bfloat16, device=DEV)
    rc = k.lib.ns_decode_attention_noalloc(q.data_ptr(), kc.data_ptr(), kc.data_ptr(),
                                           pos.data_ptr(), out.data_ptr(), Hq, Hk, D, max_len,
                                           None)
    assert rc == -2
