"""Benchmark of the MI355X quantization hot path (one GPU).

Prints ONE JSON line.  Legs:
* gru  — QuantGRU bidirectional QAT forward+backward at BASELINE config c3
         (B=256, T=200, I=80, H=256): seq/s (the headline ``value`` once built);
* qdq  — AIMET QuantizeDequantize forward+backward at config c2 ([8192, 8192] fp32,
         learnable min/max encodings, 8-bit asymmetric per-tensor and 4-bit symmetric
         per-channel): algorithmic HBM GB/s.

The roofline object describes the dominant kernel of the headline leg, timed with
events on the stream the kernel is launched on.  The CPU baseline times the CPU oracle
on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT / "rx-met_amd", ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "QuantGRU/LSTM QAT fwd+bwd seq/s (B256,T200,H256) + fake-quant HBM GB/s"
HBM_PEAK_GBS = 8000.0


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _qdq_leg(torch, steps: int, warmup: int):
    """c2: learnable-encoding QDQ fwd+bwd on [8192, 8192] (both encodings of c2)."""
    import numpy as np

    import aimet_affine as A
    import mi355x_qdq as Q
    import rxmet_lib

    dev = torch.device("cuda:0")
    R = Cc = 8192
    n = R * Cc
    torch.manual_seed(2)
    x = torch.randn(R, Cc)
    torch.manual_seed(3)
    m = torch.rand(R, Cc) < 0.01
    torch.manual_seed(4)
    x[m] = torch.randn(int(m.sum())) * 10
    torch.manual_seed(5)
    g = torch.randn(R, Cc)
    x, g = x.to(dev), g.to(dev)
    results = {}
    for name, enc_shape, bits, sym in (("per_tensor_8b_asym", (), 8, False),
                                        ("per_channel_4b_sym", (R, 1), 4, True)):
        q = A.QuantizeDequantize(enc_shape, bits, sym).to(dev)
        with q.compute_encodings():
            q(x)
        xg = x.detach().requires_grad_()

        def step():
            xg.grad = None
            q.zero_grad(set_to_none=True)
            y = q(xg)
            y.backward(g)

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        gbs = (8 + 12) * n / dt / 1e9
        results[name] = {"ms_per_step": dt * 1e3, "GB_s": gbs}
        _log(f"qdq {name}: {dt*1e3:.3f} ms/step fwd+bwd, {gbs:.0f} GB/s algorithmic")

    # Per-kernel timing of the dominant kernel (fused backward, 12 B/element) and the
    # forward, launched directly on the current stream between events.
    s_vec = torch.full((R,), 0.05, device=dev)
    o_vec = torch.zeros(R, device=dev)
    y = torch.empty_like(x)
    dx = torch.empty_like(x)
    ds = torch.empty(R, device=dev)
    do = torch.empty(R, device=dev)
    ws = torch.empty(rxmet_lib.load().rxmet_qdq_workspace_bytes(1, R, Cc), dtype=torch.uint8,
                     device=dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def fwd():
        rxmet_lib.call("rxmet_qdq_forward", x.data_ptr(), y.data_ptr(), 1, R, Cc, s_vec.data_ptr(),
                       o_vec.data_ptr(), -8, 7, Q.LEARNABLE, sh)

    def bwd():
        rxmet_lib.call("rxmet_qdq_backward", x.data_ptr(), g.data_ptr(), dx.data_ptr(),
                       ds.data_ptr(), do.data_ptr(), 1, R, Cc, s_vec.data_ptr(), o_vec.data_ptr(),
                       -8, 7, Q.LEARNABLE, ws.data_ptr(), sh)

    def ev_time(fn, reps):
        for _ in range(3):
            fn()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3

    t_f = ev_time(fwd, max(steps, 20))
    t_b = ev_time(bwd, max(steps, 20))
    results["kernel_fwd"] = {"us": t_f * 1e6, "GB_s": 8 * n / t_f / 1e9}
    results["kernel_bwd"] = {"us": t_b * 1e6, "GB_s": 12 * n / t_b / 1e9}
    _log(f"qdq kernels: fwd {t_f*1e6:.1f} us ({8*n/t_f/1e9:.0f} GB/s), "
         f"bwd {t_b*1e6:.1f} us ({12*n/t_b/1e9:.0f} GB/s)")
    roof = {"kernel": "qdq bwd_runs<LEARNABLE> (fused STE + encoding grads)", "bound": "hbm",
            "achieved": round(12 * n / t_b / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(12 * n / t_b / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
            "algorithmic_bytes_per_launch": 12 * n}
    return results, roof


def _qdq_cpu_baseline():
    """Oracle (numpy, one thread) on a 1024-row sample of c2, fwd+bwd, GB/s formula of c2."""
    import numpy as np

    import qdq_oracle as O

    rows, cols = 1024, 8192
    rng = np.random.default_rng(2)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    g = rng.standard_normal((rows, cols)).astype(np.float32)
    s, o = O.scale_offset(np.array([-4.0], np.float32), np.array([4.2], np.float32), -128, 127,
                          False)
    layout = (1, 1, rows * cols)
    t0 = time.perf_counter()
    reps = 0
    while time.perf_counter() - t0 < 10.0 or reps < 2:
        O.qdq_learnable(x, s, o, -128, 127, layout)
        O.qdq_learnable_backward(x, g, s, o, -128, 127, layout)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    gbs = 20 * rows * cols / dt / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"c2 per-tensor 8-bit learnable QDQ fwd+bwd on a [{rows}, {cols}] slice, "
                      f"numpy oracle, {reps} reps"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the path is data-parallel by batch; "
              "multi-GPU runs are not part of it)", file=sys.stderr)
        return 2
    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    _log(f"device: {torch.cuda.get_device_name(0)}")
    qdq, roof = _qdq_leg(torch, args.steps, args.warmup)
    cpu = None if args.no_cpu_baseline else _qdq_cpu_baseline()
    per_tensor = qdq["per_tensor_8b_asym"]
    line = {
        "metric": METRIC,
        "value": round(per_tensor["GB_s"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per_tensor["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "c2: QuantizeDequantize fwd+bwd, fp32 [8192, 8192], learnable "
                               "min/max encodings, 8-bit asymmetric per-tensor"},
        "qdq": {k: {kk: round(vv, 3) for kk, vv in v.items()} for k, v in qdq.items()},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
