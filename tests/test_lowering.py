"""The gfx950 lowering the split-K reduction's ordering rests on (CPU only:
hipcc compiles a few lines for gfx950 to assembly).

The reuse path's split-K tiles store fp32 partials with relaxed agent-scope
atomic stores, wait for them (s_waitcnt vmcnt(0)) and pass a barrier, take
a ticket with a relaxed agent-scope compare-and-swap, and the last arrival
reads the partials with relaxed agent-scope atomic loads
(decode-kernel_amd/csrc/dk_kernels.hpp: take_ticket, reuse_split_finish).
That is ordered because gfx950 writes agent-scope stores through the XCD's
L2 and makes agent-scope loads miss it (the sc1 bit on both), with no L2
write-back or invalidate around the compare-and-swap. This test pins that
lowering for the toolchain in use, so a compiler that lowered these atomics
differently is caught on the CPU.
"""

from __future__ import annotations

import os
import re
import subprocess
from pathlib import Path

import pytest

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"

SNIPPET = r"""
#include <hip/hip_runtime.h>
extern "C" __global__ void split_finish_pattern(float* __restrict__ partials,
                                                unsigned long long* __restrict__ ticket,
                                                float* __restrict__ out) {
  __hip_atomic_store(&partials[threadIdx.x], 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ int last;
  if (threadIdx.x == 0) {
    unsigned long long t = 0;
    last = __hip_atomic_compare_exchange_strong(ticket, &t, 1ull, __ATOMIC_RELAXED,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (last)
    out[threadIdx.x] = __hip_atomic_load(&partials[64 + threadIdx.x], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
}
"""


@pytest.mark.skipif(not HIPCC.exists(), reason="no hipcc")
def test_agent_scope_atomics_bypass_the_l2(tmp_path):
    src = tmp_path / "pattern.hip"
    src.write_text(SNIPPET)
    asm = tmp_path / "pattern.s"
    subprocess.run([str(HIPCC), "--offload-arch=gfx950", "-O3", "--cuda-device-only", "-S",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                    str(src), "-o", str(asm)], check=True, capture_output=True, timeout=300)
    text = asm.read_text()
    body = text[text.index("split_finish_pattern:"):]
    body = body[:body.index("s_endpgm")]
    stores = re.findall(r"^\s*global_store_dword\b.*$", body, re.M)
    loads = re.findall(r"^\s*global_load_dword\b.*$", body, re.M)
    # The partial store (first) and the partial load carry sc1; the plain
    # store of the result (last) does not need to.
    assert len(stores) == 2 and " sc1" in stores[0], stores
    assert len(loads) == 1 and " sc1" in loads[0], loads
    assert re.search(r"global_atomic_cmpswap_x2", body)
    # The partial stores are waited for before the barrier.
    assert re.search(r"global_store_dword[^\n]*\n(?:.*\n)*?\s*s_waitcnt vmcnt\(0\)(?:.*\n)*?\s*s_barrier",
                     body)
    # No L2 write-back or invalidate: the relaxed form costs nothing extra.
    assert "buffer_wbl2" not in body and "buffer_inv" not in body
