"""Child process of tests/test_knobs_gpu.py: the SWARMLLM_QMATMUL_MMQ
switches are read once per process, so each setting runs in a fresh one.

Reads a JSON list of products from argv[1] ({"type", "n", "k", "rows",
"seed", "capture"}), runs each through QMatMul.forward (eagerly, or captured
as a HIP graph and replayed), and writes to argv[2] an .npz with each
product's output, the decode/matrix-core launch counts its call added and
the launcher of its last kernel (qmm_last_kernel).
"""
import json
import sys

import numpy as np
import torch

from swarmllm_amd import GgmlDType, QMatMul, QTensor, fill_normal
from swarmllm_amd._lib import lib


def product(spec):
    n, k, rows = spec["n"], spec["k"], spec["rows"]
    mm = QMatMul(QTensor.quantize(fill_normal(n * k, seed=spec["seed"], std=0.02).reshape(n, k),
                                  GgmlDType(spec["type"])))
    x = fill_normal(rows * k, seed=spec["seed"] + 1).reshape(rows, k)
    L = lib()
    if spec.get("capture"):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            mm.forward(x)  # the workspace, before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        mv0, gm0 = L.qmm_matvec_launches(), L.qmm_gemm_launches()
        with torch.cuda.graph(g, stream=s):
            y = mm.forward(x)
        mv, gm = L.qmm_matvec_launches() - mv0, L.qmm_gemm_launches() - gm0
        torch.cuda.synchronize()
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
    else:
        mv0, gm0 = L.qmm_matvec_launches(), L.qmm_gemm_launches()
        y = mm.forward(x)
        mv, gm = L.qmm_matvec_launches() - mv0, L.qmm_gemm_launches() - gm0
        torch.cuda.synchronize()
    return y.cpu().numpy(), mv, gm, L.qmm_last_kernel().decode()


def main():
    specs = json.loads(sys.argv[1])
    out = {}
    for i, spec in enumerate(specs):
        print(f"product {i}: {spec}", flush=True)
        y, mv, gm, kernel = product(spec)
        out[f"y{i}"] = y
        out[f"launches{i}"] = np.array([mv, gm], np.int64)
        out[f"kernel{i}"] = np.array(kernel)
    np.savez(sys.argv[2], **out)
    print("done", flush=True)


if __name__ == "__main__":
    main()
