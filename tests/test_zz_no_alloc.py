"""The attention entry point that allocates nothing (cudallm_launch_attention_static) against the workspace one
(cudallm_launch_attention), bit for bit, through the C ABI: two calls in a row on one stream, the second with a
smaller context and a smaller max_seq (so its partial layout differs from the first call's, which the shared static
array still holds)."""
import numpy as np
import pytest

from cudallm_amd import engine as E
from oracle import kernels as K

pytestmark = pytest.mark.gpu


def _case(torch, rng, nh, nkv, max_seq, ctx):
    dev = torch.device("cuda")
    q = torch.from_numpy(rng.standard_normal(nh * 64).astype(np.float32)).to(dev)
    kc = torch.from_numpy(rng.standard_normal((nkv, max_seq, 64)).astype(np.float16)).to(dev)
    vc = torch.from_numpy(rng.standard_normal((nkv, max_seq, 64)).astype(np.float16)).to(dev)
    pos = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
    return q, kc, vc, pos


def _run_both(torch, q, kc, vc, pos, nh, nkv, max_seq):
    dev = torch.device("cuda")
    splits = max_seq // 128
    part_o = torch.empty(nh * splits * 64, dtype=torch.float32, device=dev)
    part_ml = torch.empty(nh * splits * 2, dtype=torch.float32, device=dev)
    want = torch.full((nh * 64,), float("nan"), dtype=torch.float32, device=dev)
    got = torch.full((nh * 64,), float("nan"), dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    E.launch_attention(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), part_o.data_ptr(),
                       part_ml.data_ptr(), want.data_ptr(), nh, nkv, 64, max_seq, s)
    E.launch_attention_static(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), got.data_ptr(), nh, nkv, 64,
                              max_seq, s)
    torch.cuda.synchronize()
    return got.cpu().numpy(), want.cpu().numpy()


def test_static_attention_matches_workspace_attention(gpu):
    import torch
    rng = np.random.default_rng(77)
    for nh, nkv, max_seq, ctx in ((32, 8, 8192, 8000), (32, 8, 1024, 300)):
        q, kc, vc, pos = _case(torch, rng, nh, nkv, max_seq, ctx)
        got, want = _run_both(torch, q, kc, vc, pos, nh, nkv, max_seq)
        print(f"[no-alloc] nh {nh} max_seq {max_seq} ctx {ctx}: max |static - workspace| "
              f"{float(np.max(np.abs(got - want))):.3e}", flush=True)
        np.testing.assert_array_equal(got, want)
        ref = K.attention(q.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy(), ctx, nh, nkv, 64)
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


def test_static_attention_rejects_more_than_its_slots(gpu):
    import torch
    q, kc, vc, pos = _case(torch, np.random.default_rng(1), 32, 8, 128, 1)
    with pytest.raises(E.CudaLLMError) as ei:  # 32 heads x 288 splits > 8192 slots; checked before any launch
        E.launch_attention_static(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), q.data_ptr(), 32, 8, 64,
                                  288 * 128, None)
    assert ei.value.code == 1 and "8192" in str(ei.value)


def test_static_attention_replays_under_graph_capture_and_allocates_nothing(gpu):
    """The header's two claims: the call works under HIP graph capture (captured once after a warm-up call, replayed
    three times with eager work and synchronisations in between, every replay equal to the workspace result), and
    direct calls allocate nothing (device free memory unchanged across them)."""
    import torch
    rng = np.random.default_rng(5)
    nh, nkv, max_seq, ctx = 32, 8, 1024, 700
    q, kc, vc, pos = _case(torch, rng, nh, nkv, max_seq, ctx)
    _, want = _run_both(torch, q, kc, vc, pos, nh, nkv, max_seq)  # also the warm-up call on this device
    out = torch.full((nh * 64,), float("nan"), dtype=torch.float32, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        E.launch_attention_static(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), out.data_ptr(), nh, nkv,
                                  64, max_seq, torch.cuda.current_stream().cuda_stream)
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), want, err_msg=f"graph replay {rep}")
    del g
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    s = torch.cuda.current_stream().cuda_stream
    for _ in range(4):
        E.launch_attention_static(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), out.data_ptr(), nh, nkv,
                                  64, max_seq, s)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    np.testing.assert_array_equal(out.cpu().numpy(), want)
