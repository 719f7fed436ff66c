"""The MFMA GEMM primitive (smhip_gemm) against float64 on the same (bf16-representable) inputs.

Products of bf16 values are exact in fp32 and MFMA accumulates in fp32, so the
bar is the fp32 one (1e-5 norm-wise) for fp32 output; bf16 output adds one
rounding (2e-2 bar, measures ~2e-3).  Shapes cover the fast kernel (K % 64 ==
0, both tile heights, split-K, ragged M/N edges, transposed operands) and the
generic fallback (K not a multiple of 64).  split 0 is the automatic choice the engine uses
(the 8-wave ring-buffered tile when the output has at most one 128x128 tile per CU).
"""
import numpy as np
import pytest
import torch

import sharpmind_amd
from sharpmind_amd import check

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _rnd(shape, rng):
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("M,N,K,am,bm,split", [
    (256, 256, 256, 2, 2, 1), (4096, 1024, 1024, 2, 3, 1), (300, 136, 192, 2, 3, 1), (4096, 48, 1024, 2, 3, 8),
    (48, 1024, 4096, 3, 3, 8), (1000, 32, 2048, 3, 3, 13), (8192, 512, 128, 2, 2, 1), (130, 200, 100, 2, 2, 1),
    (64, 64, 64, 0, 1, 1), (4096, 1024, 1024, 2, 2, 0), (300, 136, 192, 2, 2, 0), (130, 1000, 64, 2, 2, 0),
    (2048, 2048, 8192, 2, 2, 0), (4096, 3072, 1024, 2, 2, 0), (1000, 3072, 320, 2, 2, 0),
    # row-contiguous operands staged as stored and read transposed: the weight-gradient shapes
    # (auto split), ragged edges, the 256x192 and 256x256 tiles with a row-contiguous B
    (4096, 1024, 4096, 3, 3, 0), (1024, 2048, 4096, 3, 3, 0), (1000, 200, 320, 3, 3, 2), (600, 192, 256, 3, 3, 1),
    (4096, 3072, 1024, 2, 3, 0), (4096, 2048, 1024, 2, 3, 0), (2048, 4096, 512, 2, 3, 0), (520, 328, 448, 2, 3, 0)])
@pytest.mark.parametrize("c_bf16", [0, 1])
def test_gemm_modes(dev, M, N, K, am, bm, split, c_bf16):
    rng = np.random.default_rng(M + N + K + am + bm)
    a = _rnd((M, K), rng)
    b = _rnd((N, K), rng)
    c0 = _rnd((M, N), rng)
    dt = torch.bfloat16 if am >= 2 else torch.float32
    ta = torch.from_numpy(np.ascontiguousarray(a if am % 2 == 0 else a.T)).to(dev).to(dt)
    dtb = torch.bfloat16 if bm >= 2 else torch.float32
    tb = torch.from_numpy(np.ascontiguousarray(b if bm % 2 == 0 else b.T)).to(dev).to(dtb)
    lda = K if am % 2 == 0 else M
    ldb = K if bm % 2 == 0 else N
    for beta in (0.0, 1.0):
        tc = torch.from_numpy(c0).to(dev).to(torch.bfloat16 if c_bf16 else torch.float32)
        check(sharpmind_amd.lib().smhip_gemm(M, N, K, am, ta.data_ptr(), lda, bm, tb.data_ptr(), ldb, 0.5, beta,
                                             tc.data_ptr(), N, c_bf16, split, 1, torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        ref = 0.5 * (a.astype(np.float64) @ b.astype(np.float64).T) + beta * c0
        tol = 2e-2 if c_bf16 else 1e-5
        assert rel_err(tc.float().cpu().numpy(), ref) <= tol, (beta, rel_err(tc.float().cpu().numpy(), ref))


@pytest.mark.parametrize("qtype", [8, 12])
@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("M,N,K", [(300, 256, 512), (4096, 512, 256), (64, 1024, 768), (1000, 768, 256), (256, 256, 4096),
                                   (1024, 16384, 256), (1536, 12544, 256), (1024, 16384, 64), (2048, 8192, 128)])
def test_qgemm_bf16(orc, dev, qtype, trans, M, N, K):
    """Dequant-fused GEMM through Q8_0 / Q4_K weights, both directions (forward rows and
    the dX column planes; Q8_0 as fragment planes decoded in LDS), against float64 on the
    bf16-rounded bit-exact dequantised weights.  (256, 256, 4096) has fewer output tiles than
    CUs, so it runs split-K (fp32 partials, ordered reduction).  The last four have at least four
    tiles per CU and take the persistent form (K tiles of consecutive output tiles in one
    pipeline; K = 64 and 128 have fewer K tiles per output tile than the copy ring is deep)."""
    if qtype == 12 and (N if trans else K) % 256:
        pytest.skip("Q4_K blocks are 256 weights along the quantised axis")
    rng = np.random.default_rng(M + N + K + qtype + trans)
    shape = (K, N) if trans else (N, K)
    w = (rng.standard_normal(shape) * 0.05).astype(np.float32).ravel()
    if qtype == 8:
        raw = np.zeros(w.size // 32 * 34, np.uint8)
        assert orc.orc_quantize_q8_0(w, w.size, raw) == 0
        deq = np.zeros_like(w)
        orc.orc_dequant_q8_0(raw, deq, w.size)
    else:
        raw = np.zeros(w.size // 256 * 144, np.uint8)
        assert orc.orc_quantize_q4k(w, w.size, raw) == 0
        deq = np.zeros_like(w)
        orc.orc_dequant_q4k(raw, deq, w.size)
    wb = torch.from_numpy(deq).to(torch.bfloat16).float().numpy().reshape(shape).astype(np.float64)
    a = _rnd((M, K), rng)
    ta = torch.from_numpy(a).to(dev).to(torch.bfloat16)
    tc = torch.zeros(M, N, device=dev)
    check(sharpmind_amd.lib().smhip_qgemm_bf16(qtype, trans, M, N, K, ta.data_ptr(), K,
                                               torch.from_numpy(raw).to(dev).data_ptr(), tc.data_ptr(), N,
                                               torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ref = a.astype(np.float64) @ (wb if trans else wb.T)
    assert rel_err(tc.cpu().numpy(), ref) <= 1e-5, rel_err(tc.cpu().numpy(), ref)


def _quant(orc, qtype, w):
    if qtype == 8:
        raw = np.zeros(w.size // 32 * 34, np.uint8)
        assert orc.orc_quantize_q8_0(w, w.size, raw) == 0
        deq = np.zeros_like(w)
        orc.orc_dequant_q8_0(raw, deq, w.size)
    else:
        raw = np.zeros(w.size // 256 * 144, np.uint8)
        assert orc.orc_quantize_q4k(w, w.size, raw) == 0
        deq = np.zeros_like(w)
        orc.orc_dequant_q4k(raw, deq, w.size)
    return raw, deq


@pytest.mark.parametrize("qtype", [8, 12])
@pytest.mark.parametrize("trans,b2_mode", [(0, 3), (1, 2)])
@pytest.mark.parametrize("M,N,K,K2", [(300, 256, 512, 48), (1024, 16384, 256, 16), (1536, 12544, 512, 32),
                                      (2048, 8192, 256, 64)])
def test_qgemm_bf16_lora(orc, dev, qtype, trans, b2_mode, M, N, K, K2):
    """The adapted projection in one product, C = A deq(W)^T + s A2 B2^T (LoRALayer.Forward with
    A2 = x A): the rank operand rides as one extra K tile.  The first shape runs one output tile
    per workgroup (extension first); the others have at least four tiles per CU and take the
    persistent form, where the extension is the last K tile of each output tile and is staged by
    the decoder waves.  Forward form with the reference's B [rank, out] layout, dX form with the
    k-contiguous A operand, both base formats; float64 reference on bf16-rounded operands."""
    if qtype == 12 and (N if trans else K) % 256:
        pytest.skip("Q4_K blocks are 256 weights along the quantised axis")
    rng = np.random.default_rng(M + N + K + K2 + qtype + trans)
    shape = (K, N) if trans else (N, K)
    raw, deq = _quant(orc, qtype, (rng.standard_normal(shape) * 0.05).astype(np.float32).ravel())
    wb = torch.from_numpy(deq).to(torch.bfloat16).float().numpy().reshape(shape).astype(np.float64)
    a = _rnd((M, K), rng)
    a2 = _rnd((M, K2), rng)
    b2 = _rnd((N, K2), rng)  # B2^T rows
    s2 = 0.5  # the engine scales A2 by alpha/rank when staging it in bf16: a power of two is exact
    ta, ta2 = (torch.from_numpy(x).to(dev).to(torch.bfloat16) for x in (a, a2))
    tb2 = torch.from_numpy(np.ascontiguousarray(b2 if b2_mode == 2 else b2.T)).to(dev).to(torch.bfloat16)
    ldb2 = K2 if b2_mode == 2 else N
    tc = torch.zeros(M, N, device=dev)
    check(sharpmind_amd.lib().smhip_qgemm_bf16_lora(qtype, trans, M, N, K, ta.data_ptr(), K,
                                                    torch.from_numpy(raw).to(dev).data_ptr(), K2, ta2.data_ptr(), K2,
                                                    b2_mode, tb2.data_ptr(), ldb2, s2, tc.data_ptr(), N,
                                                    torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ref = a.astype(np.float64) @ (wb if trans else wb.T) + s2 * (a2.astype(np.float64) @ b2.astype(np.float64).T)
    assert rel_err(tc.cpu().numpy(), ref) <= 1e-5, rel_err(tc.cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,am,bm", [(6144, 32, 4096, 3, 3), (4096, 48, 4096, 2, 2), (1024, 16, 4096, 3, 3),
                                         (48, 4096, 4096, 2, 2), (4096, 48, 1024, 2, 3), (4100, 16, 3072, 2, 3),
                                         (4096, 32, 6144, 2, 2), (2000, 64, 1152, 2, 2), (16, 1000, 640, 2, 2),
                                         (4096, 16, 1024, 2, 2), (1000, 32, 1152, 2, 2)])
def test_skinny_split_reduction_repeatable(dev, M, N, K, am, bm):
    """Rank-sized products split K across workgroups (split-K partial planes, or the waves of a
    row-block workgroup when the large operand is k-contiguous) and add the splits in a fixed
    order: back-to-back calls on one stream give the same bits, and each matches float64.  The
    row-block cases cover a k-contiguous small operand (read from memory) and a [K][n] one
    (staged in LDS, read transposed), ragged M, and the rank-as-M form (output transposed)."""
    rng = np.random.default_rng(M + N)
    a = _rnd((M, K), rng)
    b = _rnd((N, K), rng)
    c0 = _rnd((M, N), rng)
    ta = torch.from_numpy(np.ascontiguousarray(a if am % 2 == 0 else a.T)).to(dev).to(torch.bfloat16)
    tb = torch.from_numpy(np.ascontiguousarray(b if bm % 2 == 0 else b.T)).to(dev).to(torch.bfloat16)
    lda = K if am % 2 == 0 else M
    ldb = K if bm % 2 == 0 else N
    ref = 0.25 * (a.astype(np.float64) @ b.astype(np.float64).T) + c0
    outs = []
    for _ in range(3):
        tc = torch.from_numpy(c0).to(dev)
        check(sharpmind_amd.lib().smhip_gemm(M, N, K, am, ta.data_ptr(), lda, bm, tb.data_ptr(), ldb, 0.25, 1.0,
                                             tc.data_ptr(), N, 0, 0, 1, torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        outs.append(tc.cpu().numpy())
        assert rel_err(outs[-1], ref) <= 1e-5
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])
