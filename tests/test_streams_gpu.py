"""Products of one weight on two streams at once: each stream gets its own
workspace (the activation's quantized planes and a K-split GEMM's slots),
so concurrent calls give exactly the results of the same calls run one
after another. Covers the few-row kernels (8 rows), the single-pass GEMM cut
along K (512 rows, its slots in the workspace) and the shared and GLU
forms."""
import pytest
import torch

from swarmllm_amd import GgmlDType, QMatMul, QTensor, fill_normal, forward_glu

pytestmark = pytest.mark.gpu


def qmm(n, k, t, seed):
    return QMatMul(QTensor.quantize(fill_normal(n * k, seed=seed, std=0.02).reshape(n, k), t))


@pytest.mark.parametrize("rows", [8, 512])
@pytest.mark.parametrize("t", [GgmlDType.Q4K, GgmlDType.Q8_0], ids=lambda t: t.name)
def test_two_streams_share_a_weight(rows, t):
    n, k = 4096, 4096
    mm = qmm(n, k, t, 930)
    other = qmm(1024, k, t, 931)
    xs = [fill_normal(rows * k, seed=940 + i).reshape(rows, k) for i in range(2)]
    want = [mm.forward(x) for x in xs]
    want_shared = [QMatMul.forward_shared(x, [mm, other]) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    got, got_shared = [[], []], [[], []]
    for _ in range(6):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                got[i].append(mm.forward(xs[i]))
                got_shared[i].append(QMatMul.forward_shared(xs[i], [mm, other]))
    torch.cuda.synchronize()
    for i in range(2):
        for y, ys in zip(got[i], got_shared[i]):
            assert torch.equal(y, want[i])
            assert torch.equal(ys[0], want_shared[i][0]) and torch.equal(ys[1], want_shared[i][1])


def test_two_streams_glu():
    k = 4096
    g, u = qmm(2048, k, GgmlDType.Q4K, 950), qmm(2048, k, GgmlDType.Q4K, 951)
    xs = [fill_normal(16 * k, seed=952 + i).reshape(16, k) for i in range(2)]
    want = [forward_glu(x, g, u) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    got = [[], []]
    for _ in range(6):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                got[i].append(forward_glu(xs[i], g, u))
    torch.cuda.synchronize()
    for i in range(2):
        assert all(torch.equal(y, want[i]) for y in got[i])
