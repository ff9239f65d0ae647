"""Benchmark of the MI355X quantization hot path (one GPU).

Prints ONE JSON line.  Legs:
* gru  — QuantGRU bidirectional QAT forward+backward at config c3
         (B=256, T=200, I=80, H=256): seq/s, the headline ``value``;
* lstm — QuantLSTM unidirectional QAT forward+backward at config c4 (B=512, T=100, I=64,
         H=512, 8-bit per-channel weights, 8-bit gates, 16-bit cell, 8-bit h): seq/s;
* qdq  — AIMET QuantizeDequantize forward+backward at config c2 ([8192, 8192] fp32,
         learnable min/max encodings, 8-bit asymmetric per-tensor and 4-bit symmetric
         per-channel): algorithmic HBM GB/s.

The roofline object describes the dominant kernel of the headline leg, timed with
hipEvents that the library records around its own launches on the stream they run on
(rxmet_prof_*), over the timed region.  The CPU baseline times the CPU oracle on a
bounded sample of the same workload (``qdq_*`` keys: the same for the QDQ leg).
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


TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic.json"


def _traffic(kernel: str):
    """HBM bytes per launch of an instrumented kernel, from the committed counter summary
    (rocprofv3 FETCH_SIZE and WRITE_SIZE passes, each scaled by what the counter reads for a
    plain copy of known size), or None when the kernel was not measured."""
    try:
        rec = json.loads(TRAFFIC_FILE.read_text())["kernels"].get(kernel)
    except (OSError, ValueError, KeyError):
        return None
    return None if rec is None else int(rec["fetch_bytes"] + rec["write_bytes"])


def _copy_probe(torch, mib: int) -> None:
    """One elementwise pass (read N bytes, write N bytes) over a buffer of `mib` MiB: the
    reference kernel that scales the HBM byte counters of a profiling run."""
    n = mib * (1 << 20) // 4
    a = torch.ones(n, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(3):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    _log(f"copy probe: 3 x neg over {mib} MiB")


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
            "frac": round(12 * n / t_b / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": _traffic("qdq_bwd_learnable"),
            "algorithmic_bytes_per_launch": 12 * n}
    return results, roof


# Algorithmic work per launch of the instrumented GRU kernels (one direction, c3 shapes):
# GEMM FLOPs 2*M*N*K as counted for the metric; the int8 MFMA / fp32 peaks are MI355X's
# published dense figures in TFLOP/s (int8: TOP/s).
INT8_MFMA_PEAK = 5000.0
FP32_MFMA_PEAK = 157.3


def _gru_kernel_work(B, T, I, H, D=2):
    """Algorithmic FLOPs per step of the instrumented c3 kernels (D directions): GEMM FLOPs
    2*M*N*K as counted for the metric; peaks are MI355X's dense figures in TFLOP/s."""
    C = 3 * H
    M = T * B
    return {
        "gru_fwd_recurrence": (D * 2.0 * M * H * C, INT8_MFMA_PEAK,
                               "recurrent GEMM R_q.h_q over T steps, both directions in one "
                               "clustered launch (int8 MFMA, 16-bit h as two byte planes)"),
        "gru_bwd_recurrence": (D * 2.0 * M * H * C, FP32_MFMA_PEAK,
                               "dh GEMM R_deq.dq over T steps, both directions in one clustered "
                               "launch (fp32 MFMA)"),
        "gru_bwd_weight_gemms": (D * 2.0 * M * C * (2 * I + H), FP32_MFMA_PEAK,
                                 "dx, dW, dR GEMMs (float gradient split into three bf16 "
                                 "terms against exact bf16 code planes, MFMA)"),
        "gru_fwd_input_gemm": (D * 2.0 * M * C * I, FP32_MFMA_PEAK,
                               "input projection W_q.x_q exact integer GEMM"),
    }


def _gru_leg(torch, steps: int, warmup: int):
    """c3: QuantGRU bidirectional QAT fwd+bwd, B=256, T=200, I=80, H=256."""
    import quant_gru as QG
    import rxmet_lib

    dev = torch.device("cuda:0")
    B, T, I, H = 256, 200, 80, 256
    torch.manual_seed(6)
    x = torch.randn(B, T, I)
    m = QG.QuantGRU(I, H, batch_first=True, bidirectional=True)  # U(+-1/16) like nn.GRU
    m.set_all_bitwidth(8, is_symmetric=False)  # weights stay symmetric, per-channel
    m._bitwidth_config.h_ = 16
    m = m.to(dev)
    x = x.to(dev)
    with m.calibration_context():
        m(x)
    m.use_quantization = True
    m.train()

    def step():
        m.zero_grad(set_to_none=True)
        out, _ = m(x)
        out.mean().backward()

    dt, p50, p95, kernels, roof = _timed_steps(torch, step, steps, warmup,
                                               _gru_kernel_work(B, T, I, H))
    total = sum(k["ms_per_step"] for k in kernels.values())
    _log(f"gru c3: {dt*1e3:.2f} ms/step wall, P50 {p50:.2f} ms P95 {p95:.2f} ms, "
         f"{B/dt:.1f} seq/s; instrumented kernels {total:.2f} ms/step")
    for k, v in sorted(kernels.items(), key=lambda kv: -kv[1]["ms_per_step"]):
        _log(f"  {k}: {v['ms_per_step']:.3f} ms/step, {v['us_per_launch']:.1f} us/launch")
    res = {"ms_per_step": dt * 1e3, "p50_ms": p50, "p95_ms": p95, "seq_per_s": B / dt,
           "seq_per_s_p50": B / (p50 * 1e-3),
           "kernels_ms_per_step": {k: round(v["ms_per_step"], 4) for k, v in kernels.items()},
           "kernels_us_per_launch": {k: round(v["us_per_launch"], 2) for k, v in kernels.items()}}
    return res, roof, m, x


def _gru_c5_leg(torch, steps: int, warmup: int):
    """c5 (a parity configuration, timed on request): QuantGRU unidirectional QAT fwd+bwd,
    B=1024, T=50, I=256, H=1024, 4-bit symmetric per-channel W_ih/W_hh, 16-bit activations
    and hidden state, power-of-2 scales."""
    import quant_gru as QG

    dev = torch.device("cuda:0")
    B, T, I, H = 1024, 50, 256, 1024
    torch.manual_seed(9)
    x = torch.randn(T, B, I)
    m = QG.QuantGRU(I, H)
    m.set_all_bitwidth(16, is_symmetric=False)
    m._bitwidth_config.W_ = 4
    m._bitwidth_config.R_ = 4
    m.use_po2_scale = True
    m = m.to(dev)
    x = x.to(dev)
    with m.calibration_context():
        m(x)
    m.use_quantization = True
    m.train()

    def step():
        m.zero_grad(set_to_none=True)
        out, _ = m(x)
        out.mean().backward()

    dt, p50, p95, kernels, _ = _timed_steps(torch, step, steps, warmup,
                                            _gru_kernel_work(B, T, I, H, D=1))
    _log(f"gru c5: {dt*1e3:.2f} ms/step wall, P50 {p50:.2f} ms, {B/dt:.1f} seq/s")
    for k, v in sorted(kernels.items(), key=lambda kv: -kv[1]["ms_per_step"]):
        _log(f"  {k}: {v['ms_per_step']:.3f} ms/step, {v['us_per_launch']:.1f} us/launch")
    return {"ms_per_step": dt * 1e3, "p50_ms": p50, "seq_per_s": B / dt,
            "kernels_ms_per_step": {k: round(v["ms_per_step"], 4) for k, v in kernels.items()}}


def _lstm_kernel_work(B, T, I, H):
    """Algorithmic FLOPs per step of the instrumented c4 kernels (one direction)."""
    C = 4 * H
    M = T * B
    return {
        "lstm_fwd_recurrence": (2.0 * M * H * C, INT8_MFMA_PEAK,
                                "recurrent GEMM W_hh_q.h_q over T steps (int8 MFMA) with the "
                                "fused gate / cell / hidden fake-quant"),
        "lstm_bwd_recurrence": (2.0 * M * H * C, INT8_MFMA_PEAK,
                                "dh GEMM W_hh_q^T.dgates over T steps (int8 MFMA, 3 planes of "
                                "22-bit block fixed point) with the fused STE pointwise"),
        "lstm_bwd_weight_gemms": (2.0 * M * C * (2 * I + H), FP32_MFMA_PEAK,
                                  "dx, dW_ih, dW_hh GEMMs (float gradient split into three "
                                  "bf16 terms against exact bf16 code planes, MFMA)"),
        "lstm_fwd_input_gemm": (2.0 * M * C * I, FP32_MFMA_PEAK,
                                "input linear W_ih_q.x_q exact integer GEMM"),
    }


def _timed_steps(torch, step, steps, warmup, work):
    """Run warmup + timed steps; per-step events, per-kernel library timings, roofline of the
    dominant instrumented kernel.

    Inside the timed region only the recurrences (the kernels the roofline can name) are
    bracketed by the library's events: every timed launch adds two event records to the
    stream, and timing all of them slows the step by about 3 %.  The per-kernel table comes
    from a second pass of the same number of steps with every launch timed."""
    import rxmet_lib

    dev = torch.device("cuda:0")
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    timed = sorted(k for k in work if "recurrence" in k)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    rxmet_lib.prof_filter(timed)
    rxmet_lib.prof_reset()
    rxmet_lib.prof_enable(True)
    t0 = time.perf_counter()
    evs[0].record(stream)
    for i in range(steps):
        step()
        evs[i + 1].record(stream)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    rxmet_lib.prof_enable(False)
    per = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(steps))
    p50 = per[len(per) // 2]
    p95 = per[min(len(per) - 1, int(0.95 * len(per)))]

    def collect():
        out = {}
        for name in rxmet_lib.prof_names():
            ms, n = rxmet_lib.prof_query(name)
            if n == 0:
                continue
            out[name] = {"ms_per_step": ms / steps, "launches_per_step": n / steps,
                         "us_per_launch": ms / max(n, 1) * 1e3}
        return out

    live = collect()
    # second pass: every instrumented launch timed, for the per-kernel table
    rxmet_lib.prof_filter(None)
    rxmet_lib.prof_reset()
    rxmet_lib.prof_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    rxmet_lib.prof_enable(False)
    kernels = collect()
    rxmet_lib.prof_reset()
    dom = max((k for k in live if k in work), key=lambda k: live[k]["ms_per_step"])
    flops_step, peak, what = work[dom]
    flops = flops_step / live[dom]["launches_per_step"]
    achieved = flops / (live[dom]["us_per_launch"] * 1e-6) / 1e12
    roof = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 3), "peak": peak,
            "unit": "TFLOP/s", "frac": round(achieved / peak, 6), "traffic": _traffic(dom),
            "algorithmic_flops_per_launch": flops, "work": what,
            "us_per_launch": round(live[dom]["us_per_launch"], 2)}
    return dt, p50, p95, kernels, roof


def _lstm_leg(torch, steps: int, warmup: int):
    """c4: QuantLSTM unidirectional QAT fwd+bwd, B=512, T=100, I=64, H=512."""
    import quant_lstm as QL

    dev = torch.device("cuda:0")
    B, T, I, H = 512, 100, 64, 512
    torch.manual_seed(7)
    x = torch.rand(T, B, I) * 2 - 1
    torch.manual_seed(8)
    g = torch.randn(T, B, H) * 0.1
    m = QL.QuantLSTM(I, H, quant_config={"schema_version": 1,
                                         "operators": {"cell_state": {"bitwidth": 16}}})
    m = m.to(dev)
    x, g = x.to(dev), g.to(dev)
    m.calibrating = True
    with torch.no_grad():
        m(x)
    m.calibrating = False
    m.finalize_calibration()
    m.use_quantization = True
    m.train()

    def step():
        m.zero_grad(set_to_none=True)
        out, _ = m(x)
        out.backward(g)

    dt, p50, p95, kernels, roof = _timed_steps(torch, step, steps, warmup,
                                               _lstm_kernel_work(B, T, I, H))
    total = sum(k["ms_per_step"] for k in kernels.values())
    _log(f"lstm c4: {dt*1e3:.2f} ms/step wall, P50 {p50:.2f} ms P95 {p95:.2f} ms, "
         f"{B/dt:.1f} seq/s; instrumented kernels {total:.2f} ms/step")
    for k, v in sorted(kernels.items(), key=lambda kv: -kv[1]["ms_per_step"]):
        _log(f"  {k}: {v['ms_per_step']:.3f} ms/step, {v['us_per_launch']:.1f} us/launch")
    res = {"ms_per_step": dt * 1e3, "p50_ms": p50, "p95_ms": p95, "seq_per_s": B / dt,
           "seq_per_s_p50": B / (p50 * 1e-3),
           "kernels_ms_per_step": {k: round(v["ms_per_step"], 4) for k, v in kernels.items()},
           "kernels_us_per_launch": {k: round(v["us_per_launch"], 2) for k, v in kernels.items()}}
    return res, roof, m, x, g


def _lstm_cpu_baseline(m, x, g, rows: int = 8):
    """CPU oracle (C, one thread) on the first `rows` sequences of c4: the q-carrier forward
    in the reference CPU path's activation semantics (glibc expf/tanhf) plus the STE
    backward, with the module's own grids."""
    import lstm_oracle as LO

    xs = x[:, :rows].detach().contiguous().cpu().numpy()
    gs = g[:, :rows].detach().contiguous().cpu().numpy()
    Wi, Wh, bi, bh = (p.detach().cpu().numpy() for p in m._direction_params(False))
    p = m._params[0].struct
    t0 = time.perf_counter()
    fwd = LO.forward_quant(Wi, Wh, bi, bh, xs, p, mode=LO.ACT_LIBM)
    t1 = time.perf_counter()
    LO.backward_quant(fwd, p, gs)
    dt = time.perf_counter() - t0
    T, Bs, I = xs.shape
    return {"value": round(Bs / dt, 3), "unit": "seq/s", "cores": 1, "kind": "port",
            "sample": f"c4 QAT fwd+bwd on {Bs} of the 512 sequences (T={T}, I={I}, "
                      f"H={m.hidden_size}), C oracle, one thread, {dt:.1f} s "
                      f"(forward {t1 - t0:.1f} s)"}


def _gru_cpu_baseline(m, x, rows: int = 32):
    """CPU oracle (C, one thread) on the first `rows` sequences of c3: the same QAT
    forward+backward of both directions with the module's own grids."""
    import numpy as np

    import gru_oracle as GO

    xs = x[:rows].detach().transpose(0, 1).contiguous().cpu().numpy()  # [T, rows, I]
    T, Bs, I = xs.shape
    H = m.hidden_size
    dirs = []
    for d, qp in enumerate((m.quant_params, m.quant_params_reverse)):
        sfx = "_reverse" if d else ""
        p = lambda n: getattr(m, n + sfx).detach().cpu().numpy()

        def swap(t):
            r, z, n = np.split(t, 3, axis=0)
            return np.concatenate([z, r, n], 0)

        W = np.ascontiguousarray(swap(p("weight_ih_l0")).T)
        R = np.ascontiguousarray(swap(p("weight_hh_l0")).T)
        dirs.append((W, R, swap(p("bias_ih_l0")), swap(p("bias_hh_l0")), qp.struct,
                     np.ascontiguousarray(xs[::-1]) if d else xs))
    gscale = np.float32(1.0 / (x.shape[0] * T * 2 * H))
    dh = np.zeros((T + 1, Bs, H), np.float32)
    dh[1:] = gscale
    t0 = time.perf_counter()
    for W, R, bw, br, qp, xd in dirs:
        fwd = GO.forward_quant(W, R, bw, br, xd, qp, training=True)
        GO.backward_quant(fwd, dh, qp)
    dt = time.perf_counter() - t0
    return {"value": round(Bs / dt, 3), "unit": "seq/s", "cores": 1, "kind": "port",
            "sample": f"c3 QAT fwd+bwd of both directions on {Bs} of the 256 sequences "
                      f"(T={T}, I={I}, H={H}), C oracle, one thread, {dt:.1f} s"}


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
    ap.add_argument("--legs", default="gru,lstm,qdq",
                    help="comma-separated subset of gru,lstm,qdq,c5 (profiling runs); the "
                         "default record runs gru, lstm and qdq")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run a plain elementwise copy over MIB MiB (scales HBM byte "
                         "counters in profiling runs)")
    args = ap.parse_args()
    legs = set(args.legs.split(","))
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the path is data-parallel by batch; "
              "multi-GPU runs are not part of it)", file=sys.stderr)
        return 2
    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    _log(f"device: {torch.cuda.get_device_name(0)}")
    if args.copy_probe:
        _copy_probe(torch, args.copy_probe)
    gru = roof = lstm = lstm_roof = qdq = qdq_roof = c5 = None
    if "gru" in legs:
        gru, roof, m, x = _gru_leg(torch, args.steps, args.warmup)
    if "lstm" in legs:
        lstm, lstm_roof, lm, lx, lg = _lstm_leg(torch, args.steps, args.warmup)
    if "qdq" in legs:
        qdq, qdq_roof = _qdq_leg(torch, args.steps, args.warmup)
    if "c5" in legs:
        c5 = _gru_c5_leg(torch, args.steps, args.warmup)
    cpu = cpu_qdq = cpu_lstm = None
    if not args.no_cpu_baseline:
        if gru is not None:
            cpu = _gru_cpu_baseline(m, x)
            _log(f"cpu baseline: {cpu}")
        if lstm is not None:
            cpu_lstm = _lstm_cpu_baseline(lm, lx, lg)
            _log(f"lstm cpu baseline: {cpu_lstm}")
        if qdq is not None:
            cpu_qdq = _qdq_cpu_baseline()
    rnd = lambda d: None if d is None else {k: (round(v, 4) if isinstance(v, float) else v)
                                            for k, v in d.items()}
    line = {
        "metric": METRIC,
        "value": round(gru["seq_per_s"], 2) if gru else None,
        "unit": "seq/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gru["ms_per_step"], 4) if gru else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "c3: QuantGRU bidirectional QAT forward+backward, B=256, T=200, "
                               "I=80, H=256, batch_first, 8-bit per-channel symmetric weights, "
                               "8-bit asymmetric activations, 16-bit h, MinMax calibration, "
                               "loss = mean(output)",
                   "batch": 256, "seq_len": 200, "input_size": 80, "hidden_size": 256,
                   "carrier": "fp32 codes; recurrent GEMMs on int8 MFMA"},
        "gru": rnd(gru),
        "lstm": rnd(lstm),
        **({"gru_c5": rnd(c5)} if c5 is not None else {}),
        "qdq": None if qdq is None else {k: {kk: round(vv, 3) for kk, vv in v.items()}
                                         for k, v in qdq.items()},
        "roofline": roof,
        "lstm_roofline": lstm_roof,
        "qdq_roofline": qdq_roof,
        "cpu_baseline": cpu,
        "lstm_cpu_baseline": cpu_lstm,
        "qdq_cpu_baseline": cpu_qdq,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
