"""Small-M products on the wide kernel: 128 x 128 tiles where 256 x 256 tiles would leave most of
the device idle (the same bits either way), split-K where the workspace entry points are given a
workspace and the tiles still leave compute units idle; the int32 row-scale path gives the same
bits as the unsplit kernel, the fp32 group-scale path matches the oracle and the unsplit kernel
closely."""
import numpy as np
import pytest
import torch

from kitchen_amd import _lib, ops
from oracle import gemm, quant

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_workspace_policy(gpu_device):
    print("[splitk] workspace policy", flush=True)
    lib = _lib.load()
    assert lib.mq_gemm_workspace_bytes(256, 3072, 3072) > 0          # 48 tiles of 128
    assert lib.mq_gemm_workspace_bytes(256, 3072, 12288) > 0
    assert lib.mq_gemm_workspace_bytes(1024, 3072, 3072) == 0        # 192 tiles of 128: no split
    assert lib.mq_gemm_workspace_bytes(4096, 12288, 3072) == 0       # 768 tiles fill the device
    assert lib.mq_gemm_workspace_bytes(64, 3072, 3072) == 0          # the few-row kernel serves M <= 128


@pytest.mark.parametrize("m,n,k", [(256, 3072, 3072), (256, 3072, 12288), (200, 1000, 3072), (300, 384, 14336)])
def test_rowscale_split_equals_unsplit(gpu_device, m, n, k):
    print(f"[splitk] rowscale M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(m + n + k)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sa = rng.uniform(0.001, 0.01, m).astype(np.float32)
    ws = rng.uniform(0.001, 0.01, n).astype(np.float32)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(gpu_device)
    qa_d, qw_d, sa_d, ws_d = _t(qa, gpu_device), _t(qw, gpu_device), _t(sa, gpu_device), _t(ws, gpu_device)
    y_split = ops.gemm_rowscale(qa_d, sa_d, qw_d, ws_d, bias, n, 8)
    y_plain = torch.empty_like(y_split)
    _lib.call("mq_gemm_rowscale", qa_d.data_ptr(), k, sa_d.data_ptr(), qw_d.data_ptr(), k, 8, ws_d.data_ptr(),
              bias.data_ptr(), _lib.DT_BF16, y_plain.data_ptr(), _lib.DT_BF16, n, m, n, k, _lib.stream_of(qa_d))
    torch.cuda.synchronize()
    assert torch.equal(y_split, y_plain)
    acc = gemm.partials(qa, qw, k)[0].astype(np.float64)
    ref = acc * sa.astype(np.float64)[:, None] * ws.astype(np.float64)[None, :] + bias.float().cpu().numpy()[None, :]
    assert gemm.rel_l2(ref, y_split.float().cpu().numpy()) < 4e-3


@pytest.mark.parametrize("m,n,k", [(256, 3072, 3072), (256, 3072, 12288), (200, 1000, 3072)])
def test_group_split_matches_oracle(gpu_device, m, n, k):
    print(f"[splitk] w4 group M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(m * 3 + n + k)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    q = rng.integers(0, 16, (n, k)).astype(np.uint8)
    z = rng.integers(0, 16, (n, k // 64)).astype(np.uint8)
    s16 = rng.uniform(1e-3, 4e-3, (n, k // 64)).astype(np.float16)
    sa = rng.uniform(0.001, 0.01, m).astype(np.float32)
    qa_d, sa_d = _t(qa, gpu_device), _t(sa, gpu_device)
    qw_d, z_d, s_d = _t(quant.pack_u4(q), gpu_device), _t(quant.pack_u4(z), gpu_device), _t(s16, gpu_device)
    y_split = ops.gemm_w4_group(qa_d, sa_d, qw_d, s_d, z_d, None, n)
    y_plain = torch.empty_like(y_split)
    _lib.call("mq_gemm_w4_group", qa_d.data_ptr(), k, sa_d.data_ptr(), qw_d.data_ptr(), k // 2, s_d.data_ptr(),
              k // 64, z_d.data_ptr(), z_d.stride(0), 64, 0, None, _lib.DT_BF16, y_plain.data_ptr(), _lib.DT_BF16, n,
              m, n, k,
              _lib.stream_of(qa_d))
    torch.cuda.synchronize()
    p = gemm.partials(qa, gemm.zero_adjusted(q, z, 64), 64)
    ref = gemm.epilogue_group(p, sa, s16.astype(np.float64))
    e_split = gemm.rel_l2(ref, y_split.float().cpu().numpy())
    e_plain = gemm.rel_l2(ref, y_plain.float().cpu().numpy())
    print(f"[splitk] rel L2 split {e_split:.2e} plain {e_plain:.2e}", flush=True)
    assert e_split < 4e-3 and e_plain < 4e-3
    assert gemm.rel_l2(y_plain.float().cpu().numpy(), y_split.float().cpu().numpy()) < 4e-3


@pytest.mark.parametrize("n", [4096, 12288])
def test_tail_rows_split(gpu_device, n):
    # M = 4352 against N = 4096 / 12288: 17 x 16 = 272 / 17 x 48 = 816 tiles of 256, a last wave of
    # one tile row on 256 units; that row runs as its own product on 128 tiles after the first 4096
    # rows (split along K for N = 4096, 64 tiles; unsplit for N = 12288, 192 tiles)
    m, k = 4352, 3072
    print(f"[splitk] tail rows M={m} N={n} K={k}", flush=True)
    lib = _lib.load()
    ws_bytes = lib.mq_gemm_workspace_bytes(m, n, k)
    assert ws_bytes % (256 * n * 4) == 0
    if n == 4096:
        assert ws_bytes // (256 * n * 4) >= 2
    assert lib.mq_gemm_workspace_bytes(4096, n, k) == 0
    rng = np.random.default_rng(11)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    sa = rng.uniform(0.001, 0.01, m).astype(np.float32)
    rows = np.r_[0:32, 4064:4128, m - 32:m]                      # both sides of the boundary
    bias = torch.randn(n, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(gpu_device)
    qa_d, sa_d = _t(qa, gpu_device), _t(sa, gpu_device)
    # int8 row scale: exact int32 sums, so the split output equals the unsplit one bit for bit
    qw = rng.integers(-127, 128, (n, k)).astype(np.int8)
    ws = rng.uniform(0.001, 0.01, n).astype(np.float32)
    qw_d, ws_d = _t(qw, gpu_device), _t(ws, gpu_device)
    y_split = ops.gemm_rowscale(qa_d, sa_d, qw_d, ws_d, bias, n, 8)
    y_plain = torch.empty_like(y_split)
    _lib.call("mq_gemm_rowscale", qa_d.data_ptr(), k, sa_d.data_ptr(), qw_d.data_ptr(), k, 8, ws_d.data_ptr(),
              bias.data_ptr(), _lib.DT_BF16, y_plain.data_ptr(), _lib.DT_BF16, n, m, n, k, _lib.stream_of(qa_d))
    torch.cuda.synchronize()
    assert torch.equal(y_split, y_plain)
    acc = qa[rows].astype(np.float64) @ qw.astype(np.float64).T          # exact in float64
    ref = acc * sa[rows].astype(np.float64)[:, None] * ws.astype(np.float64)[None, :] + \
        bias.float().cpu().numpy()[None, :]
    assert gemm.rel_l2(ref, y_split.float().cpu().numpy()[rows]) < 4e-3
    # uint4 group scale: fp32 slice sums, close to the unsplit kernel and to the oracle
    q = rng.integers(0, 16, (n, k)).astype(np.uint8)
    z = rng.integers(0, 16, (n, k // 64)).astype(np.uint8)
    s16 = rng.uniform(1e-3, 4e-3, (n, k // 64)).astype(np.float16)
    qw_d, z_d, s_d = _t(quant.pack_u4(q), gpu_device), _t(quant.pack_u4(z), gpu_device), _t(s16, gpu_device)
    y_split = ops.gemm_w4_group(qa_d, sa_d, qw_d, s_d, z_d, bias, n)
    y_plain = torch.empty_like(y_split)
    _lib.call("mq_gemm_w4_group", qa_d.data_ptr(), k, sa_d.data_ptr(), qw_d.data_ptr(), k // 2, s_d.data_ptr(),
              k // 64, z_d.data_ptr(), z_d.stride(0), 64, 0, bias.data_ptr(), _lib.DT_BF16, y_plain.data_ptr(),
              _lib.DT_BF16, n, m, n, k,
              _lib.stream_of(qa_d))
    torch.cuda.synchronize()
    assert gemm.rel_l2(y_plain.float().cpu().numpy(), y_split.float().cpu().numpy()) < 4e-3
    assert torch.equal(y_split[:4096], y_plain[:4096])                  # the unsplit rows are the same kernel
    wdq = ((q.reshape(n, -1, 64).astype(np.float64) - z.astype(np.float64)[..., None]) *
           s16.astype(np.float64)[..., None]).reshape(n, k)
    ref = (qa[rows].astype(np.float64) * sa[rows].astype(np.float64)[:, None]) @ wdq.T + bias.float().cpu().numpy()
    assert gemm.rel_l2(ref, y_split.float().cpu().numpy()[rows]) < 4e-3


@pytest.mark.parametrize("wk", ["u4", "i4x16", "i8"])
def test_tiles_agree_bitwise(gpu_device, wk):
    """The first 1024 rows of a product are the same bits whatever tile computes them: at N = 3072,
    M = 1024 runs 128 x 128 tiles, M = 2816 256 x 192 tiles, M = 4352 256 x 256 tiles; every output
    runs the same arithmetic in the same order."""
    n, k, sizes = 3072, 3072, (1024, 2816, 4352)
    m_big = sizes[-1]
    print(f"[splitk] tiles agree {wk} M={sizes} N={n} K={k}", flush=True)
    rng = np.random.default_rng(5)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(gpu_device)
    sa_d = _t(rng.uniform(0.001, 0.01, m_big).astype(np.float32), gpu_device)
    if wk == "i4x16":
        # activation layout 2: 16 q, negated in odd 64-column groups
        q = rng.integers(-7, 8, (m_big, k)).astype(np.int8)
        sign = np.where((np.arange(k) // 64) % 2 == 1, -1, 1).astype(np.int8)
        qa_d = _t((16 * q * sign[None, :]).astype(np.int8), gpu_device)
    else:
        qa_d = _t(rng.integers(-127, 128, (m_big, k)).astype(np.int8), gpu_device)
    ys = []
    for m in sizes:
        y = torch.empty((m, n), dtype=torch.bfloat16, device=gpu_device)
        if wk == "i8":
            qw_d = _t(np.random.default_rng(7).integers(-127, 128, (n, k)).astype(np.int8), gpu_device)
            ws_d = _t(np.random.default_rng(8).uniform(0.001, 0.01, n).astype(np.float32), gpu_device)
            _lib.call("mq_gemm_rowscale", qa_d.data_ptr(), k, sa_d.data_ptr(), qw_d.data_ptr(), k, 8, ws_d.data_ptr(),
                      bias.data_ptr(), _lib.DT_BF16, y.data_ptr(), _lib.DT_BF16, n, m, n, k, _lib.stream_of(qa_d))
        else:
            r2 = np.random.default_rng(9)
            if wk == "u4":
                qw = quant.pack_u4(r2.integers(0, 16, (n, k)).astype(np.uint8))
                z_d = _t(quant.pack_u4(r2.integers(0, 16, (n, k // 64)).astype(np.uint8)), gpu_device)
                z_ptr, z_ld, act = z_d.data_ptr(), z_d.stride(0), 0
            else:
                qw = quant.pack_i4(r2.integers(-7, 8, (n, k)).astype(np.int8))
                z_ptr, z_ld, act = None, 0, 2
            qw_d = _t(qw, gpu_device)
            s_d = _t(r2.uniform(1e-3, 4e-3, (n, k // 64)).astype(np.float16), gpu_device)
            _lib.call("mq_gemm_w4_group", qa_d.data_ptr(), k, sa_d.data_ptr(), qw_d.data_ptr(), k // 2, s_d.data_ptr(),
                      k // 64, z_ptr, z_ld, 64, act, bias.data_ptr(), _lib.DT_BF16, y.data_ptr(), _lib.DT_BF16, n,
                      m, n, k, _lib.stream_of(qa_d))
        torch.cuda.synchronize()
        ys.append(y)
    for y in ys[1:]:
        assert torch.equal(ys[0], y[:sizes[0]])
