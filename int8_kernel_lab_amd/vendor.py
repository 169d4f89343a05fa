"""Vendor-library baselines beside the dispatched kernel (the counterpart of
the reference's cuDNN comparison, README.md:76-90, scripts/sweep.py:44-56).

* MIOpen INT8 convolution: the C++ driver ``vendor_lab`` (next to this file),
  one process per case; see csrc/vendor_lab.cpp for its contract.
* hipBLASLt INT8 GEMM through ``torch._int_mm`` for layers that are a plain
  GEMM (1x1 filter, stride 1, no padding): y[M, N] = x[M, C] @ w[N, C]^T.
  Timed without the bias (performance only, like the reference's cuDNN
  column); its output plus the bias is compared element for element with
  the dispatched kernel's output on the same seeded data.

Both are comparisons, never a fallback: nothing here is on the product path.
"""
from __future__ import annotations

import csv
import subprocess
from pathlib import Path
from typing import Dict, List

HERE = Path(__file__).resolve().parent
VENDOR_DRIVER = HERE / "vendor_lab"
GEMM_CONTRACT = "hipblaslt int8 gemm (torch._int_mm) -> int32, no bias"


def is_plain_gemm(shape) -> bool:
    """A 1x1, stride-1, unpadded layer: the convolution is one GEMM."""
    return (shape.r == 1 and shape.s == 1 and shape.stride_h == 1 and shape.stride_w == 1
            and shape.pad_h == 0 and shape.pad_w == 0)


def miopen_row(configs: Path, case: str, warmup: int, iterations: int,
               driver: Path = VENDOR_DRIVER) -> Dict[str, str]:
    """Runs vendor_lab on one case and returns its CSV row (raises when the
    driver fails or MIOpen's output differs from the dispatched kernel's)."""
    cmd = [str(driver), "--config", str(configs), "--case", case, "--csv",
           "--warmup", str(warmup), "--iterations", str(iterations)]
    result = subprocess.run(cmd, text=True, capture_output=True)
    if result.returncode != 0:
        raise RuntimeError(f"{case}: vendor_lab exited with {result.returncode}:\n"
                           f"{result.stdout}{result.stderr}")
    return next(csv.DictReader(result.stdout.splitlines()))


def hipblaslt_gemm(shape, warmup: int = 20, iterations: int = 101) -> Dict[str, object]:
    """Times torch._int_mm on the plain-GEMM layer `shape` (median of
    per-launch event pairs) and checks it, plus the bias, against the
    dispatched kernel.  Returns hipblaslt_ms / hipblaslt_correct, or a
    contract saying why it did not run."""
    if not is_plain_gemm(shape):
        return {"hipblaslt_ms": "", "hipblaslt_correct": "",
                "hipblaslt_contract": "not a plain gemm (needs 1x1, stride 1, no padding)"}
    import torch

    import int8_kernel_lab_amd as lab

    if not torch.cuda.is_available():
        # also the case where the lab's library initialised the GPU first:
        # both load libamdhip64.so.7, and torch needs its own copy to be the
        # one the process loaded (import torch before the lab's first GPU call)
        return {"hipblaslt_ms": "", "hipblaslt_correct": "", "hipblaslt_contract": "no gpu"}
    x, w, b = lab.make_case_data(shape)
    m = shape.n * shape.h * shape.w
    a = torch.from_numpy(x.reshape(m, shape.c)).cuda()
    wt = torch.from_numpy(w.reshape(shape.k, shape.c)).cuda().t()  # [C, N] view
    bias = torch.from_numpy(b).cuda()
    try:
        y = torch._int_mm(a, wt)
    except RuntimeError as err:
        return {"hipblaslt_ms": "", "hipblaslt_correct": "",
                "hipblaslt_contract": f"torch._int_mm unsupported: {err}"[:200]}
    y_lab = torch.empty((m, shape.k), dtype=torch.int32, device="cuda")
    xd = torch.from_numpy(x).cuda()
    wd = torch.from_numpy(w).cuda()
    # the dispatched kernel's workspace (split-K partial sums on deep layers;
    # torch's allocations are 256-byte aligned)
    kernel = lab.dispatch(shape)
    ws_n = lab.workspace_bytes(kernel, shape)
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda") if ws_n else None
    torch.cuda.synchronize()
    lab.launch(kernel, shape, xd.data_ptr(), wd.data_ptr(), bias.data_ptr(), y_lab.data_ptr(),
               ws.data_ptr() if ws is not None else None, ws_n)
    lab.synchronize()
    if lab.wait_expired():
        raise RuntimeError(f"{kernel}: a bounded wait gave up; the output is not to be trusted")
    correct = bool(torch.equal(y + bias, y_lab))
    for _ in range(warmup):
        torch._int_mm(a, wt)
    torch.cuda.synchronize()
    times: List[float] = []
    for _ in range(iterations):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        torch._int_mm(a, wt)
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    times.sort()
    return {"hipblaslt_ms": times[len(times) // 2], "hipblaslt_correct": int(correct),
            "hipblaslt_contract": GEMM_CONTRACT}
