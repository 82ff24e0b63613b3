"""The allocation-free decode attention (gsvk_op_attn_decode_noalloc) against the entry point
that takes a caller workspace (gsvk_op_attn_decode): the same kernels, so the outputs must be
equal to the bit, on two calls in a row, the second with a smaller input (the library's scratch
array keeps the first call's partials and counters)."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def _case(rng, B, nh, lstride):
    q = rng.standard_normal((B, nh, 32)).astype(np.float32)
    k = rng.standard_normal((B, nh, lstride, 32)).astype(np.float16).view(np.uint16)
    v = rng.standard_normal((B, nh, lstride, 32)).astype(np.float16).view(np.uint16)
    begins = rng.integers(0, lstride // 8, B).astype(np.int32)
    ends = np.minimum(lstride, begins + rng.integers(lstride // 2, lstride, B)).astype(np.int32)
    ends[-1] = lstride
    return q, k, v, begins, ends


def _both(gpu, torch, q, k, v, kb, ke, max_keys):
    B, nh, _ = q.shape
    scale = float(np.float32(1.0) / np.sqrt(np.float32(32.0)))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    args = [dev(q), dev(k).view(torch.int16), dev(v).view(torch.int16), dev(kb), dev(ke), max_keys, scale]
    out_ws = torch.zeros((B, nh * 32), dtype=torch.float32, device="cuda")
    oq_ws = torch.zeros(B * nh * 32, dtype=torch.int8, device="cuda")
    od_ws = torch.zeros(B * nh, dtype=torch.float32, device="cuda")
    ws = torch.zeros(gpu.attn_workspace_bytes(B, nh, max_keys), dtype=torch.uint8, device="cuda")
    gpu.op_attn_decode(*args, out_ws, oq=oq_ws, od=od_ws, ws=ws)
    out_na = torch.full((B, nh * 32), float("nan"), dtype=torch.float32, device="cuda")
    oq_na = torch.zeros(B * nh * 32, dtype=torch.int8, device="cuda")
    od_na = torch.zeros(B * nh, dtype=torch.float32, device="cuda")
    gpu.op_attn_decode_noalloc(*args, out_na, oq=oq_na, od=od_na)
    torch.cuda.synchronize()
    got = out_na.cpu().numpy()
    assert np.array_equal(got, out_ws.cpu().numpy())
    assert np.array_equal(oq_na.cpu().numpy(), oq_ws.cpu().numpy())
    assert np.array_equal(od_na.cpu().numpy(), od_ws.cpu().numpy())
    ref = O.attn_decode_f16(q, k, v, kb, ke, np.float32(scale))
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-5
    return got


@pytest.mark.parametrize("first,second", [
    # 4 splits merged by the last workgroup (counters in the scratch array), then 2 splits
    ((2, 4, 4096), (1, 16, 3000)),
    # rows cut in chunks of 16 blocks (merged by a second launch), then one workgroup per row
    ((64, 16, 3100), (8, 16, 400)),
])
def test_noalloc_attention_equals_workspace_entry_point(gpu, first, second):
    import torch
    rng = np.random.default_rng(7100 + first[0])
    for B, nh, lstride in (first, second):
        print(f"noalloc attention B={B} nh={nh} lstride={lstride}", flush=True)
        q, k, v, kb, ke = _case(rng, B, nh, lstride)
        _both(gpu, torch, q, k, v, kb, ke, lstride)
