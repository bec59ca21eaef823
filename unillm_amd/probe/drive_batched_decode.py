"""Runs the batched-decode path alone, for counter collection: Q4_0 k = 4096,
n = 14336 and 4096, m = 16 and 64, 8 weight copies, 10 passes each.  Measurement
only (rocprofv3 --pmc ... -- python3 unillm_amd/probe/drive_batched_decode.py)."""
import os
import sys

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
from unillm_amd import Q4_0, QuantLinear  # noqa: E402

torch.cuda.set_device(0)
g = torch.Generator(device="cuda")
g.manual_seed(1)
for n in (14336, 4096):
    ws = []
    for _ in range(8):
        w = torch.empty(n, 4096, device="cuda").normal_(0, 0.02, generator=g)
        ws.append(QuantLinear.quantize(Q4_0, w))
        del w
    for m in (16, 64):
        x = torch.empty(m, 4096, device="cuda").normal_(generator=g)
        y = torch.empty(m, n, device="cuda")
        for _ in range(10):
            for ql in ws:
                ql.forward(x, out=y)
        torch.cuda.synchronize()
print("done", flush=True)
