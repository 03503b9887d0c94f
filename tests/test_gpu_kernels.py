"""GPU parity of the individual kernels through the C ABI.

* ragged packing: bit-exact against the C oracle (oracle/pack_ref.c);
* GEMM (MFMA bf16 / fp8-weight / fp32): against torch fp32 matmuls of the
  same (bf16-rounded) operands; bounds are half a bf16 ulp of the result
  for rounded outputs and 1e-5 relative for fp32;
* LayerNorm: against torch.nn.functional.layer_norm;
* varlen causal attention: against a per-game fp32 softmax(q k^T / 8) v.
"""
import ctypes as C
import math

import numpy as np
import pytest
import torch

from allie_amd import capi
from oracle import pack as opack

pytestmark = pytest.mark.gpu

L = None


@pytest.fixture(scope="module", autouse=True)
def _lib(cuda):
    global L
    L = capi.lib()
    yield


def rb(x):
    return x.to(torch.bfloat16).to(torch.float32)


def dev_pack(words, lens, max_len=512, block=16, first_block=0, max_blocks=None, capacity=None,
             pad_id=1996):
    dev = torch.device("cuda:0")
    B = len(lens)
    n = np.minimum(lens, max_len)
    T = int(n.sum())
    if max_blocks is None:
        max_blocks = (max_len + block - 1) // block
    cap = T if capacity is None else capacity
    wd = torch.from_numpy(np.ascontiguousarray(words, dtype=np.uint32).view(np.int32)).to(dev)
    ld = torch.from_numpy(np.asarray(lens, dtype=np.int32)).to(dev)
    i32 = lambda k: torch.full((max(k, 1),), -7, dtype=torch.int32, device=dev)
    out = {
        "cu_seqlens": i32(B + 1), "ids": i32(cap), "pos": i32(cap), "seq_of": i32(cap),
        "last_idx": i32(B), "blk_off": i32(B + 1), "block_table": i32(B * max_blocks),
        "slot": i32(cap), "status": i32(1),
    }
    in_off = torch.empty(max(B, 1), dtype=torch.int64, device=dev)
    rc = L.allie_pack_ragged(capi.ptr(wd), capi.ptr(ld), B, max_len, block, first_block, max_blocks, cap,
                             capi.ptr(out["cu_seqlens"]), capi.ptr(in_off), capi.ptr(out["ids"]),
                             capi.ptr(out["pos"]), capi.ptr(out["seq_of"]), capi.ptr(out["last_idx"]),
                             capi.ptr(out["blk_off"]), capi.ptr(out["block_table"]), capi.ptr(out["slot"]),
                             pad_id, capi.ptr(out["status"]), capi.stream_ptr())
    capi.check(rc, "pack")
    torch.cuda.synchronize()
    res = {k: v.cpu().numpy() for k, v in out.items()}
    res["block_table"] = res["block_table"][: B * max_blocks].reshape(B, max_blocks)
    for k in ("ids", "pos", "seq_of", "slot"):
        res[k] = res[k][:cap]
    res["cu_seqlens"] = res["cu_seqlens"][: B + 1]
    return res


def random_words(rng, lens):
    T = int(np.sum(lens))
    ids = rng.integers(0, 1997, T).astype(np.uint32)
    outcome = rng.integers(0, 3, T).astype(np.uint32) << 14
    secs = (rng.integers(0, 60, T).astype(np.uint32) + 1) << 16
    return ids | outcome | secs


@pytest.mark.parametrize("case", ["c2", "trunc", "single", "ones", "large_b"])
def test_pack_bit_exact(case):
    rng = np.random.default_rng(11)
    if case == "c2":
        lens = np.random.default_rng(2).integers(8, 401, 256).astype(np.int32)
    elif case == "trunc":
        lens = rng.integers(400, 700, 37).astype(np.int32)
    elif case == "single":
        lens = np.array([5], np.int32)
    elif case == "ones":
        lens = np.ones(1500, np.int32)
    else:
        lens = rng.integers(1, 80, 3000).astype(np.int32)
    words = random_words(rng, lens)  # ids over the whole vocab: PAD occurs in the larger cases
    got = dev_pack(words, lens, first_block=3)
    ref = opack.pack(words, lens, first_block=3)
    assert got["status"][0] == ref["status"]
    for k in ("cu_seqlens", "ids", "pos", "seq_of", "last_idx", "blk_off", "block_table", "slot"):
        np.testing.assert_array_equal(got[k], ref[k], err_msg=k)


def test_pack_status_flags():
    rng = np.random.default_rng(5)
    lens = np.array([4, 0, 6], np.int32)
    words = random_words(rng, lens)
    got = dev_pack(words, lens)
    assert got["status"][0] & 1
    lens = np.array([40, 50], np.int32)
    words = random_words(rng, lens)
    got = dev_pack(words, lens, capacity=60)  # too small: excess dropped, flagged
    assert got["status"][0] & 2
    assert (got["ids"][:40] == (words[:40] & 0x3FFF)).all()
    got = dev_pack(words, lens, max_blocks=2)  # 40 tokens need 3 blocks of 16
    assert got["status"][0] & 4
    words = (np.arange(30, dtype=np.uint32) % 1990) | (1 << 16)
    lens = np.array([10, 20], np.int32)
    assert dev_pack(words, lens)["status"][0] == 0
    words[25] = 1996 | (3 << 16)  # a PAD id inside the second game
    assert dev_pack(words, lens)["status"][0] == 8
    assert dev_pack(words, lens, pad_id=-1)["status"][0] == 0


def _gemm(A, Wt, bias, epi, wtype, out_f32=False, R=None, scale=None, wdq=None):
    M, K = A.shape
    N = Wt.shape[0]
    dev = A.device
    if epi == capi.EPI_RESID:
        C_ = None
    elif out_f32 or wtype == capi.WT_F32:
        C_ = torch.empty(M, N, dtype=torch.float32, device=dev)
    else:
        C_ = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    rc = L.allie_gemm(capi.ptr(A), capi.ptr(Wt), capi.ptr(bias), capi.ptr(scale), capi.ptr(C_), capi.ptr(R),
                      M, N, K, epi, wtype, int(out_f32), capi.ptr(wdq), capi.stream_ptr())
    capi.check(rc, "gemm")
    torch.cuda.synchronize()
    return C_


SHAPES = [(1, 256, 64), (300, 768, 256), (777, 1024, 1024), (1000, 3072, 1024), (513, 1024, 4096), (64, 4096, 1024)]
# large grids: ragged last m-tile, several rounds of blocks per CU, K of 4 k-tiles
LARGE_SHAPES = [(4100, 4096, 256), (16400, 1024, 512), (8192, 3072, 128)]


@pytest.mark.parametrize("M,N,K", SHAPES + LARGE_SHAPES)
def test_gemm_bf16_epilogues(M, N, K, cuda):
    g = torch.Generator(device="cpu").manual_seed(M * 7 + N + K)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16).to(cuda)
    Wt = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).to(cuda)
    b = rb(torch.randn(N, generator=g) * 0.1).to(cuda)
    acc = A.float() @ Wt.float().T + b
    # store
    C_ = _gemm(A, Wt, b, capi.EPI_STORE, capi.WT_BF16).float()
    assert ((C_ - acc).abs() <= acc.abs() * 2 ** -8 + 1e-5).all()
    # fp32 output (heads)
    C32 = _gemm(A, Wt, b, capi.EPI_STORE, capi.WT_BF16, out_f32=True)
    torch.testing.assert_close(C32, acc, rtol=1e-5, atol=1e-4)
    # gelu
    Cg = _gemm(A, Wt, b, capi.EPI_GELU, capi.WT_BF16).float()
    t = rb(acc)
    ref = (0.5 * t) * (1 + torch.tanh(math.sqrt(2 / math.pi) * (t + 0.044715 * t ** 3)))
    assert ((Cg - ref).abs() <= ref.abs() * 2 ** -6 + 2e-3).all()
    # residual
    R0 = torch.randn(M, N, generator=g).to(cuda)
    R = R0.clone()
    _gemm(A, Wt, b, capi.EPI_RESID, capi.WT_BF16, R=R)
    assert ((R - (R0 + acc)).abs() <= acc.abs() * 2 ** -8 + 1e-5).all()


# Large-M shapes of the persistent 256 x 256 kernel (store and gelu epilogues):
# several tiles per block, a ragged last m-tile, K of 2 and 16 k-tiles of 64.
# The first three leave a last round of tiles at most half full on 256 CUs,
# whose rows then run on the 128-row kernel; the fourth fills whole rounds.
PERSISTENT_SHAPES = [(20000, 1024, 1024), (53205 // 4, 3072, 128), (9000, 4096, 256), (16380, 1024, 512)]


@pytest.mark.parametrize("M,N,K", PERSISTENT_SHAPES)
@pytest.mark.parametrize("with_bias", [True, False])
def test_gemm_persistent_tiles(M, N, K, with_bias, cuda):
    g = torch.Generator(device="cpu").manual_seed(M + N * 3 + K)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16).to(cuda)
    Wt = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).to(cuda)
    b = rb(torch.randn(N, generator=g) * 0.1).to(cuda) if with_bias else None
    acc = A.float() @ Wt.float().T + (b if with_bias else 0)
    C_ = _gemm(A, Wt, b, capi.EPI_STORE, capi.WT_BF16).float()
    assert ((C_ - acc).abs() <= acc.abs() * 2 ** -8 + 1e-5).all()
    Cg = _gemm(A, Wt, b, capi.EPI_GELU, capi.WT_BF16).float()
    t = rb(acc)
    ref = (0.5 * t) * (1 + torch.tanh(math.sqrt(2 / math.pi) * (t + 0.044715 * t ** 3)))
    assert ((Cg - ref).abs() <= ref.abs() * 2 ** -6 + 2e-3).all()
    # a second call into the same buffer gives the same bits
    C2 = _gemm(A, Wt, b, capi.EPI_STORE, capi.WT_BF16).float()
    assert torch.equal(C2, C_)


def _gemm_split(A, Wt, bias, epi, wtype, split, out_f32=False, R=None, scale=None):
    M, K = A.shape
    N = Wt.shape[0]
    s = split if split > 0 else L.allie_gemm_split_factor(M, N, K)
    part = torch.empty(max(s, 1) * M * N, dtype=torch.float32, device=A.device)
    C_ = None
    if epi != capi.EPI_RESID:
        C_ = torch.empty(M, N, dtype=torch.float32 if out_f32 else torch.bfloat16, device=A.device)
    rc = L.allie_gemm_splitk(capi.ptr(A), capi.ptr(Wt), capi.ptr(bias), capi.ptr(scale), capi.ptr(C_),
                             capi.ptr(R), M, N, K, epi, wtype, int(out_f32), split, capi.ptr(part),
                             part.numel() * 4, capi.stream_ptr())
    capi.check(rc, "gemm_splitk")
    torch.cuda.synchronize()
    return C_


# (M, N, K, split): 0 = the forward's own choice (4 at M = 1024 and 8 at
# M = 63 for the MLP c_proj, see test_capi.py), ragged last m-tile, the
# heads' fp32 output
SPLIT_CASES = [(1024, 1024, 4096, 0), (63, 1024, 4096, 0), (300, 3072, 1024, 4), (1000, 1024, 1024, 2),
               (256, 2048, 1024, 4), (77, 512, 2048, 16)]


@pytest.mark.parametrize("M,N,K,split", SPLIT_CASES)
def test_gemm_split_k(M, N, K, split, cuda):
    """K-split partial sums plus the reduction pass, against the same torch
    fp32 reference and bars as the unsplit GEMM; repeated calls are bit-identical."""
    g = torch.Generator(device="cpu").manual_seed(M + N + K + split)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16).to(cuda)
    Wt = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).to(cuda)
    b = rb(torch.randn(N, generator=g) * 0.1).to(cuda)
    acc = A.float() @ Wt.float().T + b
    C_ = _gemm_split(A, Wt, b, capi.EPI_STORE, capi.WT_BF16, split).float()
    assert ((C_ - acc).abs() <= acc.abs() * 2 ** -8 + 1e-5).all()
    C2 = _gemm_split(A, Wt, b, capi.EPI_STORE, capi.WT_BF16, split).float()
    assert torch.equal(C_, C2)
    C32 = _gemm_split(A, Wt, b, capi.EPI_STORE, capi.WT_BF16, split, out_f32=True)
    torch.testing.assert_close(C32, acc, rtol=1e-5, atol=1e-4)
    Cg = _gemm_split(A, Wt, b, capi.EPI_GELU, capi.WT_BF16, split).float()
    t = rb(acc)
    ref = (0.5 * t) * (1 + torch.tanh(math.sqrt(2 / math.pi) * (t + 0.044715 * t ** 3)))
    assert ((Cg - ref).abs() <= ref.abs() * 2 ** -6 + 2e-3).all()
    R0 = torch.randn(M, N, generator=g).to(cuda)
    R = R0.clone()
    _gemm_split(A, Wt, b, capi.EPI_RESID, capi.WT_BF16, split, R=R)
    assert ((R - (R0 + acc)).abs() <= acc.abs() * 2 ** -8 + 1e-5).all()
    # fp8 weights
    w = torch.randn(N, K, generator=g) * 0.05
    s = (w.abs().amax(1) / 448.0).float()
    q = (w / s[:, None]).to(torch.float8_e4m3fn)
    accq = A.float() @ (q.float() * s[:, None]).to(cuda).T + b
    Cq = _gemm_split(A, q.view(torch.uint8).to(cuda), b, capi.EPI_STORE, capi.WT_FP8, split,
                     scale=s.to(cuda)).float()
    assert ((Cq - accq).abs() <= accq.abs() * 2 ** -8 + 1e-4).all()


@pytest.mark.parametrize("M,N", [(1000, 128), (4100, 4096)])
def test_gemm_epilogue_rounds_to_nearest_even(M, N, cuda):
    """The bf16 epilogues round fp32 sums to nearest even, bit for bit: A's
    row m carries a two-way bf16 split of x_m (hi + lo == x_m exactly, x_m
    having 16 significant bits) against weight ones, so the fp32 sum is
    exactly x_m in any summation order, and the stored bf16 must equal
    torch's RNE conversion of x_m; half of the x_m sit exactly halfway
    between two bf16 values."""
    rng = np.random.default_rng(11)
    K = 32
    bits = rng.integers(0x3A800000, 0x44800000, M, dtype=np.int64) & ~0xFF  # ~1e-3 .. 1e3
    bits[::2] = (bits[::2] & ~0xFFFF) | 0x8000  # ties
    sign = np.where(rng.random(M) < 0.5, np.int64(1) << 31, 0)
    x = torch.from_numpy((bits | sign).astype(np.uint32).view(np.float32).copy())
    hi = rb(x)
    lo = x - hi
    assert torch.equal(rb(lo), lo) and torch.equal(hi + lo, x) and not torch.equal(hi, x)
    A = torch.zeros(M, K)
    A[:, 0], A[:, 1] = hi, lo
    A = A.to(torch.bfloat16).to(cuda)
    Wt = torch.zeros(N, K)
    Wt[:, :2] = 1.0
    Wt = Wt.to(torch.bfloat16).to(cuda)
    want = x.to(torch.bfloat16)[:, None].expand(M, N)
    zero_bias = torch.zeros(N, device=cuda)
    for b in (None, zero_bias):
        C_ = _gemm(A, Wt, b, capi.EPI_STORE, capi.WT_BF16).cpu()
        assert torch.equal(C_.view(torch.int16), want.contiguous().view(torch.int16))
        R = torch.zeros(M, N, device=cuda)
        _gemm(A, Wt, b, capi.EPI_RESID, capi.WT_BF16, R=R)
        assert torch.equal(R.cpu(), want.float())
        C32 = _gemm(A, Wt, b, capi.EPI_STORE, capi.WT_BF16, out_f32=True).cpu()
        assert torch.equal(C32, x[:, None].expand(M, N))


@pytest.mark.parametrize("M,N,K", [(300, 768, 256), (1000, 3072, 1024), (4100, 4096, 256)])
def test_gemm_fp8_weights(M, N, K, cuda):
    g = torch.Generator(device="cpu").manual_seed(N + K)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16).to(cuda)
    w = torch.randn(N, K, generator=g) * 0.05
    s = (w.abs().amax(1) / 448.0).float()
    q = (w / s[:, None]).to(torch.float8_e4m3fn)
    deq = q.float() * s[:, None]
    b = rb(torch.randn(N, generator=g) * 0.1).to(cuda)
    qd, sd = q.view(torch.uint8).to(cuda), s.to(cuda)
    acc = A.float() @ deq.to(cuda).T + b
    C_ = _gemm(A, qd, b, capi.EPI_STORE, capi.WT_FP8, scale=sd).float()
    assert ((C_ - acc).abs() <= acc.abs() * 2 ** -8 + 1e-4).all()
    R0 = torch.randn(M, N, generator=g).to(cuda)
    R = R0.clone()
    _gemm(A, qd, b, capi.EPI_RESID, capi.WT_FP8, R=R, scale=sd)
    assert ((R - (R0 + acc)).abs() <= acc.abs() * 2 ** -8 + 1e-4).all()
    # with a widening buffer the weights are widened to bf16 first (exactly);
    # below the persistent kernel's size the same products are summed in the
    # same order: the same bits
    wdq = torch.empty(N, K, dtype=torch.bfloat16, device=cuda)
    same = -(-M // 256) * (N // 256) < 256
    Cw = _gemm(A, qd, b, capi.EPI_STORE, capi.WT_FP8, scale=sd, wdq=wdq).float()
    assert torch.equal(Cw, C_) if same else ((Cw - acc).abs() <= acc.abs() * 2 ** -8 + 1e-4).all()
    Rw = R0.clone()
    _gemm(A, qd, b, capi.EPI_RESID, capi.WT_FP8, R=Rw, scale=sd, wdq=wdq)
    assert torch.equal(Rw, R)
    if same:
        Cg = _gemm(A, qd, b, capi.EPI_GELU, capi.WT_FP8, scale=sd).float()
        Cgw = _gemm(A, qd, b, capi.EPI_GELU, capi.WT_FP8, scale=sd, wdq=wdq).float()
        assert torch.equal(Cgw, Cg)


@pytest.mark.parametrize("M,N,K", PERSISTENT_SHAPES)
def test_gemm_fp8_weights_persistent(M, N, K, cuda):
    """Large M with a widening buffer: the fp8 weights are widened to bf16
    and the persistent kernel scales in the epilogue; same bars as the
    256x128 kernel's fp8 path, store and gelu, bias on and off."""
    g = torch.Generator(device="cpu").manual_seed(N + K + 1)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16).to(cuda)
    w = torch.randn(N, K, generator=g) * 0.05
    s = (w.abs().amax(1) / 448.0).float()
    q = (w / s[:, None]).to(torch.float8_e4m3fn)
    deq = q.float() * s[:, None]
    qd, sd = q.view(torch.uint8).to(cuda), s.to(cuda)
    wdq = torch.empty(N, K, dtype=torch.bfloat16, device=cuda)
    for with_bias in (True, False):
        b = rb(torch.randn(N, generator=g) * 0.1).to(cuda) if with_bias else None
        acc = A.float() @ deq.to(cuda).T + (b if with_bias else 0)
        C_ = _gemm(A, qd, b, capi.EPI_STORE, capi.WT_FP8, scale=sd, wdq=wdq).float()
        assert ((C_ - acc).abs() <= acc.abs() * 2 ** -8 + 1e-4).all(), (with_bias, (C_ - acc).abs().max())
        Cg = _gemm(A, qd, b, capi.EPI_GELU, capi.WT_FP8, scale=sd, wdq=wdq).float()
        t = rb(acc)
        ref = (0.5 * t) * (1 + torch.tanh(math.sqrt(2 / math.pi) * (t + 0.044715 * t ** 3)))
        assert ((Cg - ref).abs() <= ref.abs() * 2 ** -6 + 2e-3).all(), (with_bias, (Cg - ref).abs().max())
    # the widened weights are the exact fp8 values
    assert torch.equal(wdq.float(), q.float().to(cuda))


# skinny path (M <= 8 rows): the row counts of its three register variants
# and their edges, one and four waves per workgroup (N < 2048), the medium
# and 2x model's projection shapes, the heads' fp32 output (N = 2048), K not
# a multiple of one step (512 or 2048 elements), and the first M past the
# skinny range (the MFMA path)
SKINNY_SHAPES = [(1, 3072, 1024), (2, 1024, 4096), (4, 4096, 1024), (5, 5120, 1280), (8, 2048, 1024),
                 (7, 1024, 1024), (6, 1280, 5120), (3, 64, 8), (1, 1280, 1280), (9, 1024, 1024)]


@pytest.mark.parametrize("M,N,K", SKINNY_SHAPES)
def test_gemm_skinny_rows(M, N, K, cuda):
    """M <= 8: the skinny kernel, every epilogue, bf16 and fp8 weights,
    against the torch fp32 reference with the bars of the MFMA kernels;
    repeated calls are bit-identical."""
    g = torch.Generator(device="cpu").manual_seed(M * 13 + N + K)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16).to(cuda)
    Wt = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).to(cuda)
    b = rb(torch.randn(N, generator=g) * 0.1).to(cuda)
    acc = A.float() @ Wt.float().T + b
    C_ = _gemm(A, Wt, b, capi.EPI_STORE, capi.WT_BF16).float()
    assert ((C_ - acc).abs() <= acc.abs() * 2 ** -8 + 1e-5).all()
    assert torch.equal(_gemm(A, Wt, b, capi.EPI_STORE, capi.WT_BF16).float(), C_)
    C_nb = _gemm(A, Wt, None, capi.EPI_STORE, capi.WT_BF16).float()
    acc_nb = acc - b
    assert ((C_nb - acc_nb).abs() <= acc_nb.abs() * 2 ** -8 + 1e-5).all()
    C32 = _gemm(A, Wt, b, capi.EPI_STORE, capi.WT_BF16, out_f32=True)
    torch.testing.assert_close(C32, acc, rtol=1e-5, atol=1e-4)
    Cg = _gemm(A, Wt, b, capi.EPI_GELU, capi.WT_BF16).float()
    t = rb(acc)
    ref = (0.5 * t) * (1 + torch.tanh(math.sqrt(2 / math.pi) * (t + 0.044715 * t ** 3)))
    assert ((Cg - ref).abs() <= ref.abs() * 2 ** -6 + 2e-3).all()
    R0 = torch.randn(M, N, generator=g).to(cuda)
    R = R0.clone()
    _gemm(A, Wt, b, capi.EPI_RESID, capi.WT_BF16, R=R)
    assert ((R - (R0 + acc)).abs() <= acc.abs() * 2 ** -8 + 1e-5).all()
    w = torch.randn(N, K, generator=g) * 0.05
    s = (w.abs().amax(1) / 448.0).float()
    q = (w / s[:, None]).to(torch.float8_e4m3fn)
    accq = A.float() @ (q.float() * s[:, None]).to(cuda).T + b
    qd, sd = q.view(torch.uint8).to(cuda), s.to(cuda)
    Cq = _gemm(A, qd, b, capi.EPI_STORE, capi.WT_FP8, scale=sd).float()
    assert ((Cq - accq).abs() <= accq.abs() * 2 ** -8 + 1e-4).all()
    Rq = R0.clone()
    _gemm(A, qd, b, capi.EPI_RESID, capi.WT_FP8, R=Rq, scale=sd)
    assert ((Rq - (R0 + accq)).abs() <= accq.abs() * 2 ** -8 + 1e-4).all()


@pytest.mark.parametrize("M,N,K", [(1, 256, 64), (300, 770, 256), (129, 2048, 1024)])
def test_gemm_fp32(M, N, K, cuda):
    g = torch.Generator(device="cpu").manual_seed(N * 3 + K)
    A = torch.randn(M, K, generator=g).to(cuda)
    Wt = (torch.randn(N, K, generator=g) * 0.05).to(cuda)
    b = (torch.randn(N, generator=g) * 0.1).to(cuda)
    acc = (A.double() @ Wt.double().T + b.double()).float()
    C_ = _gemm(A, Wt, b, capi.EPI_STORE, capi.WT_F32)
    torch.testing.assert_close(C_, acc, rtol=1e-5, atol=1e-5)
    Cg = _gemm(A, Wt, b, capi.EPI_GELU, capi.WT_F32)
    torch.testing.assert_close(Cg, torch.nn.functional.gelu(acc, approximate="tanh"), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("bf16", [True, False])
def test_layernorm(bf16, cuda):
    g = torch.Generator(device="cpu").manual_seed(3)
    d = 1024
    h = (torch.randn(100, d, generator=g) * 3 + 1).to(cuda)
    gam = (1 + 0.1 * torch.randn(d, generator=g)).to(cuda)
    bet = (0.1 * torch.randn(d, generator=g)).to(cuda)
    idx = torch.tensor([5, 99, 0, 42], dtype=torch.int32, device=cuda)
    y = torch.empty(6, d, dtype=torch.bfloat16 if bf16 else torch.float32, device=cuda)
    rc = L.allie_layernorm(capi.ptr(h), capi.ptr(idx), 4, 6, d, capi.ptr(gam), capi.ptr(bet), 1e-5, capi.ptr(y),
                           int(bf16), capi.stream_ptr())
    capi.check(rc)
    torch.cuda.synchronize()
    ref = torch.nn.functional.layer_norm(h[idx.long()], (d,), gam, bet, 1e-5)
    tol = 2 ** -8 if bf16 else 1e-5
    assert ((y[:4].float() - ref).abs() <= ref.abs() * tol + 1e-5).all()
    assert (y[4:].float() == 0).all()


def _tiles(lens, qt=64):
    nt = [(n + qt - 1) // qt for n in lens]
    out = []
    for q in range(max(nt) - 1, -1, -1):
        out += [(s << 5) | q for s in range(len(lens)) if nt[s] > q]
    return out


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("H", [4, 16])
def test_attention_varlen(bf16, H, cuda):
    lens = [1, 2, 5, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200, 300, 400, 511, 512]
    if H == 16 and not bf16:
        lens = lens[:12]
    d = H * 64
    T = sum(lens)
    g = torch.Generator(device="cpu").manual_seed(H)
    qkv = torch.randn(T, 3 * d, generator=g) * 1.5
    if bf16:
        qkv = rb(qkv)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    tiles = _tiles(lens)
    dt = torch.bfloat16 if bf16 else torch.float32
    qkv_d = qkv.to(dt).to(cuda)
    out = torch.full((T, d), float("nan"), dtype=dt, device=cuda)
    cu_d = torch.from_numpy(cu).to(cuda)
    tiles_d = torch.tensor(tiles, dtype=torch.int32, device=cuda)
    order_ws = torch.empty(len(lens), dtype=torch.int32, device=cuda)
    rc = L.allie_attn_varlen(capi.ptr(qkv_d), capi.ptr(cu_d), capi.ptr(tiles_d), len(tiles), len(lens), T, H, 64,
                             0.125, capi.ptr(out), int(bf16), capi.ptr(order_ws), capi.stream_ptr())
    capi.check(rc)
    torch.cuda.synchronize()
    out = out.float().cpu()
    for s, n in enumerate(lens):
        x = qkv[cu[s]: cu[s + 1]]
        q, k, v = x.split(d, dim=1)
        q = q.view(n, H, 64).transpose(0, 1)
        k = k.view(n, H, 64).transpose(0, 1)
        v = v.view(n, H, 64).transpose(0, 1)
        sc = (q @ k.transpose(1, 2)) * 0.125
        sc = sc.masked_fill(~torch.ones(n, n, dtype=torch.bool).tril(), float("-inf"))
        ref = (torch.softmax(sc, -1) @ v).transpose(0, 1).reshape(n, d)
        got = out[cu[s]: cu[s + 1]]
        if bf16:
            torch.testing.assert_close(got, ref, rtol=2e-2, atol=2e-2)
        else:
            torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-5)
