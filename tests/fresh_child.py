"""Child process of tests/test_device_arm_gpu.py for what a process decides
once: the loader switches (SWARMLLM_LOAD_PINNED, SWARMLLM_LOAD_READ, read
once) and a product whose first call is under a HIP graph capture (the
per-device preparation, qmm_prepare).

    fresh_child.py load PATH NAME OUT.npz     load one tensor, save its bytes
    fresh_child.py capture OUT.npz            the capture sequence below

Writes an .npz the parent checks; prints each step before it runs.
"""
import sys

import numpy as np
import torch


def step(msg):
    print(msg, flush=True)


def load(path, name, out):
    from swarmllm_amd.gguf import Content, pinned_load_chunks

    c0 = pinned_load_chunks()
    step(f"load {name} from {path}")
    q = Content.read(path).tensor(name)
    torch.cuda.synchronize()
    np.savez(out, data=q.data_.cpu().numpy(), pad=q.storage_[q.data_.numel():].cpu().numpy(),
             chunks=np.array([pinned_load_chunks() - c0], np.int64))


def capture(out):
    from swarmllm_amd import GgmlDType, QMatMul, QTensor, fill_normal, prepare, prepared
    from swarmllm_amd._lib import lib

    L = lib()
    res = {}

    def last():
        return L.qmm_last_kernel().decode()

    # a Q4_K product of 4 rows against a 9.4 MB weight: the few-row
    # matrix-core kernel's case once the type is prepared
    n, k, rows = 4096, 4096, 4
    mm = QMatMul(QTensor.quantize(fill_normal(n * k, seed=91, std=0.02).reshape(n, k), GgmlDType.Q4K))
    x = fill_normal(rows * k, seed=92).reshape(rows, k)
    res["prepared_before"] = np.array([prepared(GgmlDType.Q4K)])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()

    step("capture: the first Q4_K product of the process")
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1, stream=s):
        y1 = mm.forward(x)
    res["kernel_first"] = np.array(last())
    res["prepared_after_capture"] = np.array([prepared(GgmlDType.Q4K)])
    y1.fill_(float("nan"))
    with torch.cuda.stream(s):
        g1.replay()
    torch.cuda.synchronize()
    res["y_first"] = y1.cpu().numpy()

    step("eager: the same product outside a capture (prepares Q4_K)")
    y2 = mm.forward(x)
    torch.cuda.synchronize()
    res["kernel_eager"] = np.array(last())
    res["prepared_after_eager"] = np.array([prepared(GgmlDType.Q4K)])
    res["y_eager"] = y2.cpu().numpy()

    step("capture: the product again, its type now prepared")
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s):
        y3 = mm.forward(x)
    res["kernel_second"] = np.array(last())
    for r in range(2):
        y3.fill_(float("nan"))
        with torch.cuda.stream(s):
            g2.replay()
        torch.cuda.synchronize()
        res[f"y_second{r}"] = y3.cpu().numpy()

    step("capture: a Q6_K GEMM of 512 rows whose kernel has never run")
    n6, k6, m6 = 2048, 4096, 512
    mm6 = QMatMul(QTensor.quantize(fill_normal(n6 * k6, seed=93, std=0.02).reshape(n6, k6), GgmlDType.Q6K))
    x6 = fill_normal(m6 * k6, seed=94).reshape(m6, k6)
    g3 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g3, stream=s):
        y6 = mm6.forward(x6)
    res["kernel_gemm"] = np.array(last())
    y6.fill_(float("nan"))
    with torch.cuda.stream(s):
        g3.replay()
    torch.cuda.synchronize()
    res["y_gemm_captured"] = y6.cpu().numpy()
    res["y_gemm_eager"] = mm6.forward(x6).cpu().numpy()

    step("capture: the no-allocation entry's first call, after qmm_prepare")
    n8, k8, m8 = 1024, 2048, 16
    w8 = QTensor.quantize(fill_normal(n8 * k8, seed=95, std=0.02).reshape(n8, k8), GgmlDType.Q8_0)
    x8 = fill_normal(m8 * k8, seed=96).reshape(m8, k8)
    prepare(GgmlDType.Q8_0)
    y8 = torch.empty((m8, n8), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    g4 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g4, stream=s):
        st = L.qmm_forward_noalloc(8, w8.data_.data_ptr(), x8.data_ptr(), k8, y8.data_ptr(), n8, k8, n8, m8,
                                   torch.cuda.current_stream().cuda_stream)
    res["noalloc_status"] = np.array([st])
    y8.fill_(float("nan"))
    with torch.cuda.stream(s):
        g4.replay()
    torch.cuda.synchronize()
    res["y_noalloc_captured"] = y8.cpu().numpy()
    res["y_noalloc_eager"] = QMatMul(w8).forward(x8).cpu().numpy()
    np.savez(out, **res)
    step("done")


def main():
    if sys.argv[1] == "load":
        load(sys.argv[2], sys.argv[3], sys.argv[4])
    elif sys.argv[1] == "capture":
        capture(sys.argv[2])
    else:
        raise SystemExit(f"unknown mode {sys.argv[1]}")


if __name__ == "__main__":
    main()
