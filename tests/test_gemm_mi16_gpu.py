"""GPU parity of the aligned FP32 route (256x256, 64x256 and 32x128 tiles
on v_mfma_f32_16x16x4_f32, taken when M and N are multiples of the tile
and K of one pipeline loop: 64, or 128 for the eight-stage 32x128 tile)
against the CPU oracle, with every epilogue, alpha / accumulate and
the batch-broadcast forms; shapes just off the alignment take the other
kernels and must agree too.  Tolerances as in test_gemm_gpu.check_f32.
"""

import pytest

from test_gemm_gpu import run_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=["f32_m256n256", "f32_m64n256", "f32_m32n128"])
def kex(ta, ctx, request):
    e = ta.Executor(ctx, kernel_selection=request.param, tune=False)
    yield e
    e.close()


EPIS = [dict(), dict(bias=True), dict(act=1), dict(act=2, bias=True), dict(act=3, binary=1, beta=0.5),
        dict(binary=2), dict(alpha=0.25, accumulate=True, act=3), dict(bias=True, act=2, binary=2)]


@pytest.mark.parametrize("shape", [(256, 256, 64), (256, 256, 128), (512, 768, 192), (768, 512, 1024)])
@pytest.mark.parametrize("epi", EPIS)
def test_aligned_epilogues(ta, kex, oracle, shape, epi):
    m, n, k = shape
    epi = dict(epi)
    bias = [n] if epi.pop("bias", False) else None
    run_case(ta, kex, oracle, m, n, k, bias=bias, kernel_ex=kex, **epi)


@pytest.mark.parametrize("ba,bb,bc", [(3, 1, 3), (1, 3, 3), (1, 1, 3), (3, 3, 3)])
def test_aligned_batch_broadcast(ta, kex, oracle, ba, bb, bc):
    run_case(ta, kex, oracle, 256, 512, 64, batch_a=ba, batch_b=bb, batch_c=bc, bias=[bc, 512], act=1,
             kernel_ex=kex)


@pytest.mark.parametrize("shape", [(256, 256, 48), (256, 256, 16), (256, 256, 32), (256, 256, 96),
                                   (255, 256, 64), (256, 260, 64), (512, 512, 4000)])
def test_unaligned_fall_back(ta, kex, oracle, shape):
    run_case(ta, kex, oracle, *shape, bias=[shape[1]], act=3, kernel_ex=kex)


def test_deep_k_and_repeat_determinism(ta, kex, oracle):
    """K = 8192 (512 stages) and the same result bits on a second run."""
    import numpy as np
    m, n, k = 256, 256, 8192
    ha, hb = oracle.fill_det(m * k, 401), oracle.fill_det(k * n, 402)
    a, b, c = kex.tensor_from(ha, shape=[m, k]), kex.tensor_from(hb, shape=[k, n]), kex.tensor([m, n])
    kex.run_ops([ta.MatmulOp(a, b, c)])
    first = kex.download(c)
    kex.run_ops([ta.MatmulOp(a, b, c)])
    assert np.array_equal(first, kex.download(c))
    from test_gemm_gpu import check_f32
    check_f32(first, oracle.reference_gemm(ha, hb, 1, m, n, k), k, oracle, epi=False)
