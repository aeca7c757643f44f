"""Run as a script by tests/test_gpu_parity.py::test_torch_interop_subprocess.

A caller that holds torch tensors: torch is imported first so that libvxs.so binds to torch's HIP
runtime (same soname), the context launches on torch's current stream, and the ids are checked
against the CPU oracle.
"""
import os
import sys

import torch  # noqa: E402  (must precede voxwerk_amd)

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import numpy as np  # noqa: E402

from oracle import ref  # noqa: E402
from parity import compare_ids  # noqa: E402
from voxwerk_amd import workloads  # noqa: E402
from voxwerk_amd.sampler import Context  # noqa: E402


def main() -> int:
    w = workloads.workload(3)
    b = w.generate()
    dev = torch.device("cuda:0")
    t_logits = torch.from_numpy(b.logits).to(dev)
    t_off = torch.from_numpy(b.hist_off).to(dev)
    t_hist = torch.from_numpy(b.hist_ids).to(dev)
    t_params = torch.from_numpy(b.params.view(np.uint8).copy()).to(dev)
    t_u = torch.from_numpy(b.u).to(dev)
    out = torch.empty(b.rows, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()
    with Context(0) as ctx:
        ctx.set_stream(stream.cuda_stream)
        ctx.sample_device(b.rows, w.vocab, t_logits, w.vocab, t_params, 1, t_u, out, t_off, t_hist)
        torch.cuda.synchronize()
    ids = out.cpu().numpy()
    ora = ref.sample(b.logits, b.params, b.u, b.hist_off, b.hist_ids, threads=8)
    rep = compare_ids(ids, ora)
    print(f"torch interop {w.name}: {rep}")
    return 0 if not rep.unexplained else 1


if __name__ == "__main__":
    sys.exit(main())
