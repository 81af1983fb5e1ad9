"""sinkattn_block_sparse_attn_noalloc (the forward from a bool mask with the plan in the
library's static device array) against sinkattn_block_sparse_plan + sinkattn_block_sparse_fwd
with caller buffers, both through the C ABI.

The two run the same kernels on the same plan, so the outputs must be bit-identical.  Two calls
in a row, the second on a smaller input (the static array still holds the first call's larger
plan), then the first shape again; the no-allocation path on its own against the oracle; plus
the size limit, which is checked on the host before any launch."""
import ctypes
import math

import pytest
import torch

from oracle import torch_ref
from sinkattn_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(B, H, N, dtype, seed, density):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, N, 128, generator=g).to("cuda", dtype) for _ in range(3))
    nb = math.ceil(N / 128)
    mask = torch.rand(B, H, nb, nb, generator=g) < density
    d = torch.arange(nb)
    mask[:, :, d, d] = True
    mask[0, 0, nb // 2] = False                     # one empty row
    return q, k, v, mask.cuda()


def _outputs(q):
    B, H, N, D = q.shape
    out = torch.full((B, N, H, D), float("nan"), dtype=q.dtype, device=q.device).permute(0, 2, 1, 3)
    lse = torch.full((B, H, N), float("nan"), dtype=torch.float32, device=q.device)
    return out, lse


def _noalloc(q, k, v, mask):
    out, lse = _outputs(q)
    _noalloc_into(q, k, v, mask.to(torch.uint8), out, lse)
    return out, lse


def _noalloc_into(q, k, v, m, out, lse):
    lib = _lib.lib()
    B, H, Nq, D = q.shape
    rc = lib.sinkattn_block_sparse_attn_noalloc(
        m.data_ptr(), _lib.strides4(m), q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.dtype_code(q.dtype),
        B, H, Nq, k.shape[2], D, _lib.strides4(q), _lib.strides4(k), _lib.strides4(v),
        out.data_ptr(), _lib.strides4(out), lse.data_ptr(), 1.0 / math.sqrt(D), _lib.stream_ptr(q.device))
    _lib.check(rc, "sinkattn_block_sparse_attn_noalloc")


def _with_plan(q, k, v, mask):
    lib = _lib.lib()
    B, H, Nq, D = q.shape
    Nk = k.shape[2]
    nqb, nkb = mask.shape[2], mask.shape[3]
    m = mask.to(torch.uint8)
    counts = torch.empty(B * H * nqb, dtype=torch.int32, device=q.device)
    idx = torch.empty(B * H * nqb * nkb, dtype=torch.int32, device=q.device)
    order = torch.empty(lib.sinkattn_block_sparse_order_slots(B, H, nqb), dtype=torch.int32, device=q.device)
    stream = _lib.stream_ptr(q.device)
    _lib.check(lib.sinkattn_block_sparse_plan(m.data_ptr(), _lib.strides4(m), B, H, nqb, nkb, counts.data_ptr(),
                                              idx.data_ptr(), order.data_ptr(), stream), "plan")
    out, lse = _outputs(q)
    _lib.check(lib.sinkattn_block_sparse_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.dtype_code(q.dtype), B, H, Nq, Nk, D,
        _lib.strides4(q), _lib.strides4(k), _lib.strides4(v), out.data_ptr(), _lib.strides4(out),
        lse.data_ptr(), counts.data_ptr(), idx.data_ptr(), order.data_ptr(), nqb, nkb, 1.0 / math.sqrt(D),
        stream), "fwd")
    return out, lse


def _same(a, b):
    return torch.equal(a.view(torch.int16) if a.dtype != torch.float32 else a.view(torch.int32),
                       b.view(torch.int16) if b.dtype != torch.float32 else b.view(torch.int32))


def test_noalloc_matches_plan_and_forward_twice_then_smaller():
    big = _inputs(2, 6, 3000, torch.bfloat16, seed=1, density=0.3)
    small = _inputs(1, 2, 700, torch.bfloat16, seed=2, density=0.5)
    for q, k, v, mask in (big, small, big):
        print(f"noalloc vs plan+fwd: q {tuple(q.shape)} mask {tuple(mask.shape)}", flush=True)
        got_o, got_l = _noalloc(q, k, v, mask)
        want_o, want_l = _with_plan(q, k, v, mask)
        torch.cuda.synchronize()
        assert not torch.isnan(got_o).any() and not torch.isnan(got_l).any()
        assert _same(got_o, want_o)
        assert _same(got_l, want_l)
        assert torch.isinf(got_l[0, 0, (mask.shape[2] // 2) * 128]).item()   # the empty row


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_against_the_oracle(dtype):
    """The no-allocation path checked on its own against the oracle's dense masked softmax
    (the same bars as the plan + forward parity tests: |dO| <= 2e-2 max and 1e-3 mean, fp32
    lse within 4e-3 + 1e-5 |lse|, empty rows give out = 0 and lse = +inf), then once more on a
    smaller shape after it, so the second call reads the plan the first one left behind."""
    for B, H, N, seed, density in ((1, 3, 1300, 8, 0.35), (1, 2, 500, 9, 0.6)):
        q, k, v, mask = _inputs(B, H, N, dtype, seed=seed, density=density)
        print(f"noalloc vs oracle: {dtype} q {tuple(q.shape)} mask {tuple(mask.shape)}", flush=True)
        out, lse = _noalloc(q, k, v, mask)
        torch.cuda.synchronize()
        ref_o, ref_l = torch_ref.dense_masked_attention(q, k, v, mask)
        o, l = out.float().cpu(), lse.cpu()
        err = (o - ref_o).abs()
        assert err.max().item() <= 2e-2 and err.mean().item() <= 1e-3, (err.max().item(), err.mean().item())
        fin = torch.isfinite(ref_l)
        assert torch.equal(fin, torch.isfinite(l))
        assert ((l[fin] - ref_l[fin]).abs() <= 4e-3 + 1e-5 * ref_l[fin].abs()).all()
        assert torch.equal(o[~fin], torch.zeros_like(o[~fin]))


def test_noalloc_f16_bshd_views():
    q, k, v, mask = _inputs(1, 4, 1000, torch.float16, seed=3, density=0.4)
    q, k, v = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v))
    got = _noalloc(q, k, v, mask)
    want = _with_plan(q, k, v, mask)
    torch.cuda.synchronize()
    assert _same(got[0], want[0]) and _same(got[1], want[1])


def test_noalloc_rejects_plans_beyond_the_static_buffer():
    lib = _lib.load_library()
    z = (ctypes.c_int64 * 4)(0, 0, 0, 1)
    # 2 x 40 x 591 x 591 blocks (Wan-14B 720p) needs ~112 MB of plan: refused before any launch
    rc = lib.sinkattn_block_sparse_attn_noalloc(None, z, None, None, None, 0, 2, 40, 75600, 75600, 128,
                                                z, z, z, None, z, None, 0.088, None)
    assert rc < 0
    msg = lib.sinkattn_last_error().decode()
    assert "static plan buffer" in msg and "sinkattn_block_sparse_plan" in msg


def test_noalloc_captured_in_a_graph_replays_new_inputs():
    """After one eager call on the GPU (the static buffer's address is then known), the call
    is captured with torch.cuda.graph and replayed on new q/k/v/mask contents copied into the
    captured buffers; every replay must equal plan + forward on the same inputs, bit for bit,
    with eager work and synchronisations between the replays."""
    q, k, v, mask = _inputs(1, 3, 1500, torch.bfloat16, seed=4, density=0.35)
    m = mask.to(torch.uint8)
    out, lse = _outputs(q)
    _noalloc_into(q, k, v, m, out, lse)            # eager first call
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _noalloc_into(q, k, v, m, out, lse)
    torch.cuda.synchronize()
    for seed in (5, 6, 7):
        q2, k2, v2, mask2 = _inputs(1, 3, 1500, torch.bfloat16, seed=seed, density=0.2 + 0.1 * (seed - 5))
        print(f"graph replay seed {seed}", flush=True)
        q.copy_(q2), k.copy_(k2), v.copy_(v2), m.copy_(mask2.to(torch.uint8))
        out.fill_(float("nan")), lse.fill_(float("nan"))
        g.replay()
        want_o, want_l = _with_plan(q2, k2, v2, mask2)   # eager work between replays
        torch.cuda.synchronize()
        assert not torch.isnan(out).any() and not torch.isnan(lse).any()
        assert _same(out, want_o)
        assert _same(lse, want_l)
