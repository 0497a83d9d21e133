"""The build's check of lds_copy.h's M0 invariant (swarmllm_amd/m0_check.py):
it passes the library's own kernels and fails a kernel that copies through
dma16 and also reads M0, whether the reader is added to a disassembly or
compiled into a real gfx950 object (compiled only, never run)."""
import os
import subprocess

import pytest

from swarmllm_amd import m0_check

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "swarmllm_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"

GOOD = """
0000000000001000 <copy_kernel>:
\ts_load_dwordx2 s[2:3], s[0:1], 0x0                         // 000000001000: C0060080 00000000
\ts_mov_b32 m0, s4                                           // 000000001008: BEFC0004
\ts_nop 0                                                    // 00000000100C: BF800000
\tglobal_load_lds_dwordx4 v1, s[2:3]                         // 000000001010: DDF48000 00020001
\tv_mfma_i32_32x32x32_i8 a[0:15], v[2:5], v[6:9], a[0:15]    // 000000001018: D3B60000 04020D02
\ts_endpgm                                                   // 000000001020: BF810000

0000000000002000 <other_kernel>:
\ts_sendmsg sendmsg(MSG_DEALLOC_VGPRS)                       // 000000002000: BF900000
\ts_endpgm                                                   // 000000002004: BF810000
"""


def with_line(text, after, line):
    return text.replace(after, after + "\n\t" + line, 1)


def test_disassembly_rules():
    assert m0_check.violations(GOOD) == []  # a kernel without copies may read M0
    bad = [
        with_line(GOOD, "v_mfma_i32_32x32x32_i8 a[0:15], v[2:5], v[6:9], a[0:15]", "s_mov_b32 s5, m0"),
        with_line(GOOD, "v_mfma_i32_32x32x32_i8 a[0:15], v[2:5], v[6:9], a[0:15]", "s_sendmsg sendmsg(MSG_INTERRUPT)"),
        with_line(GOOD, "v_mfma_i32_32x32x32_i8 a[0:15], v[2:5], v[6:9], a[0:15]", "v_movrels_b32 v0, v1"),
        with_line(GOOD, "v_mfma_i32_32x32x32_i8 a[0:15], v[2:5], v[6:9], a[0:15]", "ds_append v3"),
        with_line(GOOD, "v_mfma_i32_32x32x32_i8 a[0:15], v[2:5], v[6:9], a[0:15]",
                  "buffer_load_dword v1, off, s[8:11], 0 lds"),
        with_line(GOOD, "v_mfma_i32_32x32x32_i8 a[0:15], v[2:5], v[6:9], a[0:15]", "s_add_u32 s6, s6, m0"),
        # a second copy without its own M0 set
        with_line(GOOD, "v_mfma_i32_32x32x32_i8 a[0:15], v[2:5], v[6:9], a[0:15]", "global_load_lds_dword v1, s[2:3]"),
    ]
    for text in bad:
        assert len(m0_check.violations(text)) == 1, text
    assert "copy_kernel" in m0_check.violations(bad[0])[0]


TOOLS = all(os.path.exists(p) for p in (HIPCC, f"{m0_check.LLVM}/llvm-objdump",
                                        f"{m0_check.LLVM}/clang-offload-bundler", f"{m0_check.LLVM}/llvm-objcopy"))


@pytest.mark.skipif(not TOOLS, reason="needs hipcc and the ROCm LLVM tools")
def test_a_compiled_m0_reader_is_caught(tmp_path):
    src = tmp_path / "k.hip"
    src.write_text(f'''
#include "{CSRC}/lds_copy.h"
__global__ void copy_then_read(const int* g, int* out, int reader) {{
  __shared__ int buf[256];
  qmm::dma4(g, 4u * threadIdx.x, qmm::lds_addr(buf));
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int v = buf[threadIdx.x];
  if (reader) {{
#ifdef ADD_READER
    int m;
    asm volatile("s_mov_b32 %0, m0" : "=s"(m));
    v += m;
#endif
  }}
  out[threadIdx.x] = v;
}}
''')
    flags = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-c"]
    for define, expect in ((None, 0), ("-DADD_READER", 1)):
        obj = tmp_path / ("bad.o" if define else "good.o")
        cmd = [HIPCC, *flags, str(src), "-o", str(obj)] + ([define] if define else [])
        subprocess.run(cmd, check=True, capture_output=True)
        found, copying = m0_check.check_objects([str(obj)])
        assert copying == 1
        assert len(found) == expect, found


@pytest.mark.skipif(not TOOLS or not os.path.exists(os.path.join(CSRC, "_build", "gemm_q4k_sp.o")),
                    reason="needs the built objects and the ROCm LLVM tools")
def test_the_library_s_copying_kernels_hold_the_invariant():
    found, copying = m0_check.check_objects([os.path.join(CSRC, "_build", "gemm_q4k_sp.o"),
                                             os.path.join(CSRC, "_build", "gemm_q4k_skinny.o")])
    assert found == [] and copying >= 3
