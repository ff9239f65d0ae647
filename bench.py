"""Benchmark of the MI355X quantization hot path (one GPU).

Prints ONE JSON line.  Legs (all run by default):
* gru  — QuantGRU bidirectional QAT forward+backward at config c3
         (B=256, T=200, I=80, H=256): seq/s, the headline ``value``;
* lstm — QuantLSTM unidirectional QAT forward+backward at config c4 (B=512, T=100, I=64,
         H=512, 8-bit per-channel weights, 8-bit gates, 16-bit cell, 8-bit h): seq/s;
* qdq  — AIMET QuantizeDequantize forward+backward at config c2 ([8192, 8192] fp32,
         learnable min/max encodings, 8-bit asymmetric per-tensor and 4-bit symmetric
         per-channel): algorithmic HBM GB/s;
* c1   — the QuantGRU PTQ calibration pass (B=32, T=98, I=40, H=64): calibration forward,
         parameter derivation and PTQ forward, seq/s;
* c5   — QuantGRU unidirectional QAT forward+backward at B=1024, T=50, I=256, H=1024 (4-bit
         weights, 16-bit activations and h, power-of-2 scales): seq/s;
* gint — the c3 model on the int32 carrier, PTQ inference of both directions (the work the
         reference's CPU int carrier does, timed by the c3 CPU baseline), float and int-IO: seq/s;
* lstmpub — the reference's published QuantLSTM inference profiles ([50, 64, 128, 256] and
         [16, 128, 64, 128], cuda-performance.md), P50 / P95 over 200 calls, beside its numbers;
* calib — the MinMax calibration forwards at c3 (GRU, both directions), c4 (LSTM) and c5 (GRU):
         ms per calibration forward over the whole batch.

The roofline object describes the dominant kernel of the headline leg, timed with
hipEvents that the library records around its own launches on the stream they run on
(rxmet_prof_*), over the timed region.  After each leg the benchmarked outputs are checked:
every output and gradient finite, and sampled sequences equal to the CPU oracle (forward
bit-exact, dx within 1e-4); a failed check ends the run with exit status 3 and no JSON line.
The CPU baselines time the reference's own CPU code (compiled from its sources into
oracle/_ref) on a bounded sample of the same workload, with the host's CPU model stated.
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


def _qdq_leg(torch, steps: int, warmup: int, validate: bool = True):
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
    # fused: the mirror module's one-launch encodings; reference_path: the reference module's
    # get_encodings() tensor expressions before the backend call, what aimet_torch's own
    # QuantizeDequantize runs with this backend registered
    for name, enc_shape, bits, sym, fused in (
            ("per_tensor_8b_asym", (), 8, False, True),
            ("per_channel_4b_sym", (R, 1), 4, True, True),
            ("per_tensor_8b_asym_reference_path", (), 8, False, False),
            ("per_channel_4b_sym_reference_path", (R, 1), 4, True, False)):
        q = A.QuantizeDequantize(enc_shape, bits, sym).to(dev)
        q.fused_encodings = fused
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
        results[name] = {"ms_per_step": dt * 1e3, "GB_s": gbs, "frac": gbs / HBM_PEAK_GBS}
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
    # calibration min / max (the observer's pass, 4 B/element read) per tensor and per channel
    ws1 = torch.empty(rxmet_lib.load().rxmet_qdq_workspace_bytes(1, 1, n), dtype=torch.uint8,
                      device=dev)
    ws2 = torch.empty_like(ws)
    mn_out, mx_out = torch.empty(R, device=dev), torch.empty(R, device=dev)
    for nm, C_, inner_, w_ in (("kernel_minmax_per_tensor", 1, n, ws1),
                               ("kernel_minmax_per_channel", R, Cc, ws2)):
        t_m = ev_time(lambda: rxmet_lib.call("rxmet_qdq_minmax", x.data_ptr(), 1, C_, inner_,
                                             mn_out.data_ptr(), mx_out.data_ptr(),
                                             w_.data_ptr(), sh),
                      max(steps, 20))
        results[nm] = {"us": t_m * 1e6, "GB_s": 4 * n / t_m / 1e9,
                       "frac": 4 * n / t_m / 1e9 / HBM_PEAK_GBS}
    # the practical ceiling: a plain elementwise pass over the same tensor (read + write)
    y_copy = torch.empty_like(x)
    t_c = ev_time(lambda: torch.neg(x, out=y_copy), max(steps, 20))
    del y_copy, ws1, ws2
    results["copy_ceiling"] = {"us": t_c * 1e6, "GB_s": 8 * n / t_c / 1e9,
                               "frac": 8 * n / t_c / 1e9 / HBM_PEAK_GBS,
                               "what": "torch.neg over the [8192, 8192] fp32 tensor (read x, "
                                       "write y): the bandwidth a plain streaming pass reaches"}
    _log(f"qdq min/max: per tensor {results['kernel_minmax_per_tensor']['GB_s']:.0f} GB/s, "
         f"per channel {results['kernel_minmax_per_channel']['GB_s']:.0f} GB/s; copy ceiling "
         f"{results['copy_ceiling']['GB_s']:.0f} GB/s")
    results["kernel_fwd"] = {"us": t_f * 1e6, "GB_s": 8 * n / t_f / 1e9}
    results["kernel_bwd"] = {"us": t_b * 1e6, "GB_s": 12 * n / t_b / 1e9}
    _log(f"qdq kernels: fwd {t_f*1e6:.1f} us ({8*n/t_f/1e9:.0f} GB/s), "
         f"bwd {t_b*1e6:.1f} us ({12*n/t_b/1e9:.0f} GB/s)")
    # the same launches on a bf16 copy of the tensor (2 bytes per element; the 4-bit grid is
    # not stable in bf16, so the arithmetic runs in fp32 as the reference's would)
    xh, gh = x.to(torch.bfloat16), g.to(torch.bfloat16)
    yh, dxh = torch.empty_like(xh), torch.empty_like(xh)
    dsh, doh = torch.empty_like(ds), torch.empty_like(do)
    lay = rxmet_lib.QdqLayout(1, 1, 1, R, Cc)
    num = rxmet_lib.QdqNumerics(2, 0, 0.0, 0, 0)
    wsh = torch.empty(rxmet_lib.load().rxmet_qdq_workspace_bytes_ex(lay, 2), dtype=torch.uint8,
                      device=dev)

    def fwd_bf16():
        rxmet_lib.call("rxmet_qdq_forward_ex", xh.data_ptr(), yh.data_ptr(), lay, num,
                       s_vec.data_ptr(), o_vec.data_ptr(), -8, 7, Q.LEARNABLE, sh)

    def bwd_bf16():
        rxmet_lib.call("rxmet_qdq_backward_ex", xh.data_ptr(), gh.data_ptr(), dxh.data_ptr(),
                       dsh.data_ptr(), doh.data_ptr(), lay, num, s_vec.data_ptr(),
                       o_vec.data_ptr(), -8, 7, Q.LEARNABLE, wsh.data_ptr(), sh)

    t_fh = ev_time(fwd_bf16, max(steps, 20))
    t_bh = ev_time(bwd_bf16, max(steps, 20))
    results["kernel_fwd_bf16"] = {"us": t_fh * 1e6, "GB_s": 4 * n / t_fh / 1e9}
    results["kernel_bwd_bf16"] = {"us": t_bh * 1e6, "GB_s": 6 * n / t_bh / 1e9}
    _log(f"qdq kernels (bf16 tensor): fwd {t_fh*1e6:.1f} us ({4*n/t_fh/1e9:.0f} GB/s), "
         f"bwd {t_bh*1e6:.1f} us ({6*n/t_bh/1e9:.0f} GB/s)")
    del xh, gh, yh, dxh, dsh, doh, wsh
    results.update(_qc_op_timings(torch, x, ev_time, max(steps, 20)))
    check = None
    if validate:
        # the timed kernels' outputs on 64 rows against the oracle: y and dx bit-exact, the
        # per-row encoding gradients within summation-order noise
        import qdq_oracle as O

        torch.cuda.synchronize()
        rows = 64
        xs, gs = x[:rows].cpu().numpy(), g[:rows].cpu().numpy()
        sv, ov = s_vec[:rows].cpu().numpy(), o_vec[:rows].cpu().numpy()
        lay = (1, rows, Cc)
        ey, _ = O.qdq_learnable(xs, sv, ov, -8, 7, lay)
        edx, eds, edo = O.qdq_learnable_backward(xs, gs, sv, ov, -8, 7, lay)
        _check_equal("qdq forward", y[:rows].cpu().numpy(), ey)
        _check_equal("qdq dx", dx[:rows].cpu().numpy(), edx)
        e1 = _check_close("qdq dscale", ds[:rows].cpu().numpy(), eds, rtol=1e-5)
        e2 = _check_close("qdq doffset", do[:rows].cpu().numpy(), edo, rtol=1e-5)
        check = {"rows": rows, "forward": "bit-exact", "dx": "bit-exact",
                 "encoding_grad_max_abs_err_rel": max(e1, e2)}
        _log(f"c2 validation: {check}")
    roof = {"kernel": "qdq bwd_runs<LEARNABLE> (fused STE + encoding grads)", "bound": "hbm",
            "achieved": round(12 * n / t_b / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(12 * n / t_b / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": _traffic("qdq_bwd_learnable"),
            "algorithmic_bytes_per_launch": 12 * n}
    return results, roof, check


def _qc_op_timings(torch, x, ev_time, reps):
    """The ONNX Runtime op QcQuantizeOp (rxmet_qc_quantize_compute) on the c2 tensor: 8-bit
    TF encodings per tensor and per row; quantizeDequantize (read x, write y: 8 B/element) and
    oneShotQuantizeDequantize (statistics pass, encodings, quantize-dequantize: 12 B/element),
    and quantizeDequantize on a float16 copy (4 B/element).  64 rows of the one-shot result
    against the oracle, bit for bit."""
    import ctypes

    import numpy as np

    import rxmet_lib
    from qc_quantize_op import BlockTensorQuantizer, OpMode, QcQuantizeInfo

    R, Cc = x.shape
    n = R * Cc
    sh = torch.cuda.current_stream(x.device).cuda_stream
    arr = (ctypes.c_int64 * 2)(R, Cc)
    out = {}
    y = torch.empty_like(x)
    xh = x.to(torch.float16)
    yh = torch.empty_like(xh)
    for label, eshape in (("per_tensor", ()), ("per_channel", (R, 1))):
        q = BlockTensorQuantizer(eshape, 8)
        info = QcQuantizeInfo()
        info.tensorQuantizerRef = q
        c = info.c_struct

        def run(mode, src=x, dst=y, io=0):
            c.op_mode = mode
            rxmet_lib.call("rxmet_qc_quantize_compute", ctypes.byref(c), src.data_ptr(),
                           dst.data_ptr(), io, arr, 2, None, sh)

        t_one = ev_time(lambda: run(int(OpMode.oneShotQuantizeDequantize)), reps)
        if label == "per_channel":
            import qc_quantize_oracle as QO

            torch.cuda.synchronize()
            rows = np.sort(np.random.default_rng(3).choice(R, 64, replace=False))
            xs = x[rows].cpu().numpy()
            oq = QO.BlockTensorQuantizerOracle((64, 1), 8)
            oq.update_stats(xs)
            oq.set_encodings(oq.compute_encodings(False))
            _check_equal("qc oneShot per row", y[rows].cpu().numpy(), oq.quantize_dequantize(xs))
        t_q = ev_time(lambda: run(int(OpMode.quantizeDequantize)), reps)
        t_h = ev_time(lambda: run(int(OpMode.quantizeDequantize), xh, yh, 1), reps)
        for nm, t, b in (("one_shot", t_one, 12), ("qdq", t_q, 8), ("qdq_f16", t_h, 4)):
            gbs = b * n / t / 1e9
            out[f"qc_op_{nm}_{label}"] = {"us": t * 1e6, "GB_s": gbs, "frac": gbs / HBM_PEAK_GBS}
        _log(f"QcQuantizeOp {label}: oneShot {t_one*1e6:.1f} us ({12*n/t_one/1e9:.0f} GB/s), "
             f"quantizeDequantize {t_q*1e6:.1f} us ({8*n/t_q/1e9:.0f} GB/s), fp16 "
             f"{t_h*1e6:.1f} us ({4*n/t_h/1e9:.0f} GB/s)")
        del q, info
    del y, xh, yh
    return out


# Algorithmic work per launch of the instrumented GRU kernels (one direction, c3 shapes):
# GEMM FLOPs 2*M*N*K as counted for the metric, priced against the MI355X published dense peak
# of the MFMA type that executes them, in TFLOP/s (int8: TOP/s).  Float products computed as
# three exact bf16 terms against exact bf16 code planes run on bf16 MFMA: three bf16 products
# per algorithmic product, so their fraction of the bf16 peak is at most 1/3.
INT8_MFMA_PEAK = 5000.0
BF16_MFMA_PEAK = 2500.0


def _gru_kernel_work(B, T, I, H, D=2, stepped_bwd=False):
    """Algorithmic FLOPs per step of the instrumented GRU kernels (D directions): GEMM FLOPs
    2*M*N*K as counted for the metric; peaks are MI355X's dense figures in TFLOP/s."""
    C = 3 * H
    M = T * B
    dirs = "both directions in one clustered launch" if D == 2 else "one clustered launch"
    bwd = ("one direction, stepped: per time step one dh GEMM launch (bf16 MFMA: dq split into "
           "three bf16 terms against the R codes) and one pointwise launch" if stepped_bwd else
           f"{dirs} (bf16 MFMA: dq split into three bf16 terms against the R codes)")
    return {
        "gru_fwd_recurrence": (D * 2.0 * M * H * C, INT8_MFMA_PEAK,
                               f"recurrent GEMM R_q.h_q over T steps, {dirs} (int8 MFMA, 16-bit "
                               "h as two byte planes)"),
        "gru_bwd_recurrence": (D * 2.0 * M * H * C, BF16_MFMA_PEAK,
                               f"dh GEMM R_deq.dq over T steps, {bwd}"),
        "gru_bwd_weight_gemms": (D * 2.0 * M * C * (2 * I + H), BF16_MFMA_PEAK,
                                 "dx, dW, dR GEMMs (float gradient split into three bf16 "
                                 "terms against exact bf16 code planes, MFMA)"),
        "gru_fwd_input_gemm": (D * 2.0 * M * C * I, INT8_MFMA_PEAK,
                               "input projection W_q.x_q exact integer GEMM"),
    }


class ValidationError(RuntimeError):
    """The benchmarked path produced outputs that are non-finite or differ from the oracle."""


def _host_info():
    """Host CPU of the box the baselines ran on."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = None
    return {"cpu_model": model, "nproc": os.cpu_count(), "usable_cpus": usable}


def _check_close(name, got, exp, rtol=1e-4):
    import numpy as np

    if not np.isfinite(got).all():
        raise ValidationError(f"{name}: non-finite values")
    scale = max(float(np.abs(exp).max()), 1e-30)
    err = float((np.abs(got - exp) / (rtol * np.abs(exp) + 1e-5 * scale)).max())
    if err > 1.0:
        raise ValidationError(f"{name}: differs from the oracle (error {err:.3g} of the bar)")
    return float(np.abs(got - exp).max() / scale)


def _check_equal(name, got, exp):
    import numpy as np

    if not np.array_equal(got, exp):
        raise ValidationError(f"{name}: not bit-exact against the oracle "
                              f"({int((got != exp).sum())} elements differ)")


def _swap_gates(t):
    import numpy as np

    r, z, n = np.split(t, 3, axis=0)
    return np.concatenate([z, r, n], 0)


def _gru_dirs_haste(m):
    """Per direction: (W [I,3H], R [H,3H], bw, br, qparams struct, ranges, config) of a
    QuantGRU, in the kernel-side (z, r, n) layout the oracle takes."""
    import numpy as np

    out = []
    for d in range(m.num_directions):
        sfx = "_reverse" if d else ""
        p = lambda n: getattr(m, n + sfx).detach().cpu().numpy()
        qp = m.quant_params_reverse if d else m.quant_params
        rg = m.quant_ranges_reverse if d else m.quant_ranges
        out.append((np.ascontiguousarray(_swap_gates(p("weight_ih_l0")).T),
                    np.ascontiguousarray(_swap_gates(p("weight_hh_l0")).T),
                    _swap_gates(p("bias_ih_l0")), _swap_gates(p("bias_hh_l0")), qp.struct,
                    rg.to_struct(), m._bitwidth_config.to_struct()))
    return out


def _validate_gru(torch, m, x, rows, batch_first):
    """One more step of the benchmarked module (loss = mean of the output): outputs and every
    gradient finite, the sampled sequences' output (bit-exact) and dx (1e-4) equal to the
    oracle run on those sequences alone."""
    import numpy as np

    import gru_oracle as GO

    m.zero_grad(set_to_none=True)
    xl = x.detach().clone().requires_grad_(True)
    out, _ = m(xl)
    out.mean().backward()
    torch.cuda.synchronize()
    if not bool(torch.isfinite(out).all()) or not bool(torch.isfinite(xl.grad).all()):
        raise ValidationError("gru: non-finite output or input gradient")
    for name, p in m.named_parameters():
        if not bool(torch.isfinite(p.grad).all()):
            raise ValidationError(f"gru: non-finite gradient of {name}")
    H = m.hidden_size
    xt = x.detach().transpose(0, 1) if batch_first else x.detach()
    xs = xt[:, rows].contiguous().cpu().numpy()
    ot = out.detach().transpose(0, 1) if batch_first else out.detach()
    got = ot[:, rows].cpu().numpy()
    gx = xl.grad.transpose(0, 1) if batch_first else xl.grad
    gx = gx[:, rows].cpu().numpy()
    T = xs.shape[0]
    gval = np.float32(1.0 / out.numel())
    dx = np.zeros(xs.shape, np.float64)
    for d, (W, R, bw, br, qp, _, _) in enumerate(_gru_dirs_haste(m)):
        xd = np.ascontiguousarray(xs[::-1]) if d else xs
        fwd = GO.forward_quant(W, R, bw, br, xd, qp, training=True)
        o = fwd["h"][1:][::-1] if d else fwd["h"][1:]
        _check_equal(f"gru output dir{d}", got[..., d * H:(d + 1) * H], o)
        dh = np.zeros((T + 1, len(rows), H), np.float32)
        dh[1:] = gval
        bwd = GO.backward_quant(fwd, dh, qp)
        dx += bwd["dx"][::-1] if d else bwd["dx"]
    err = _check_close("gru dx", gx, dx)
    return {"sequences": list(rows), "forward": "bit-exact", "dx_max_abs_err_rel": err,
            "grads_finite": True}


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


def _gru_int_leg(torch, steps: int, warmup: int):
    """gint: the c3 model on the int32 carrier, PTQ inference (eval, no autograd) of both
    directions -- the work of the reference's quantGRUForwardCPU, which the c3 CPU baseline
    times -- with float input and output (quant_storage_dtype='int32'), and the same forward
    with int32 codes in and out (forward_quantized)."""
    import quant_gru as QG

    dev = torch.device("cuda:0")
    B, T, I, H = 256, 200, 80, 256
    torch.manual_seed(6)
    x = torch.randn(B, T, I)
    m = QG.QuantGRU(I, H, batch_first=True, bidirectional=True)
    m.set_all_bitwidth(8, is_symmetric=False)
    m._bitwidth_config.h_ = 16
    m = m.to(dev).eval()
    x = x.to(dev)
    with m.calibration_context():
        m(x)
    m.use_quantization = True
    m.quant_storage_dtype = "int32"
    out = {}

    def step():
        with torch.no_grad():
            out["y"] = m(x)[0]

    C, M = 3 * H, T * B
    work = {"gru_int_recurrence": (2.0 * M * H * C, INT8_MFMA_PEAK,
                                   "recurrent GEMM R_q (h_q - zp_h) of one direction over T steps "
                                   "(one clustered launch: int8 MFMA on h byte planes, the "
                                   "integer gates fused)"),
            "gru_int_input_gemm": (2.0 * M * C * I, INT8_MFMA_PEAK,
                                   "input projection W_q (x_q - zp_x) of one direction")}
    dt, p50, p95, kernels, roof = _timed_steps(torch, step, steps, warmup, work)
    meta = m.get_io_quant_meta()
    xin = meta["input"]
    lo = 0 if xin["is_unsigned"] else -(1 << (xin["bitwidth"] - 1))
    hi = (1 << xin["bitwidth"]) - 1 if xin["is_unsigned"] else (1 << (xin["bitwidth"] - 1)) - 1
    xq = (torch.round(x / torch.tensor(xin["scale"], device=dev)) + xin["zp"]).clamp(lo, hi)
    xq = xq.to(torch.int32)

    def step_io():
        out["q"] = m.forward_quantized(xq)[0]

    for _ in range(warmup):
        step_io()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step_io()
    torch.cuda.synchronize()
    dt_io = (time.perf_counter() - t0) / steps
    _log(f"gru int32 carrier (c3 shape, PTQ inference): {dt*1e3:.2f} ms/step, {B/dt:.1f} seq/s; "
         f"int codes in/out {dt_io*1e3:.2f} ms/step, {B/dt_io:.1f} seq/s")
    for k, v in sorted(kernels.items(), key=lambda kv: -kv[1]["ms_per_step"]):
        _log(f"  {k}: {v['ms_per_step']:.3f} ms/step, {v['us_per_launch']:.1f} us/launch")
    res = {"ms_per_step": dt * 1e3, "p50_ms": p50, "p95_ms": p95, "seq_per_s": B / dt,
           "int_io_ms_per_step": dt_io * 1e3, "int_io_seq_per_s": B / dt_io,
           "kernels_ms_per_step": {k: round(v["ms_per_step"], 4) for k, v in kernels.items()}}
    return res, roof, m, x, out


def _validate_gru_int(m, x, y, yq, rows):
    """The int32-carrier outputs of the sampled sequences equal the oracle's int32 carrier
    (which equals the reference's CPU carrier code for code), bit for bit; the int-IO output
    codes are the same h codes."""
    import numpy as np

    import gru_oracle as GO
    import rxmet_gru_abi as A

    H = m.hidden_size
    xs = x.detach().transpose(0, 1)[:, rows].contiguous().cpu().numpy()
    got = y.detach().transpose(0, 1)[:, rows].cpu().numpy()
    gq = yq.detach().transpose(0, 1)[:, rows].cpu().numpy()
    for d, (W, R, bw, br, qp, _, _) in enumerate(_gru_dirs_haste(m)):
        xd = np.ascontiguousarray(xs[::-1]) if d else xs
        f = GO.forward_int(W, R, bw, br, xd, qp, training=False)
        hq = f["h_q"][1:][::-1] if d else f["h_q"][1:]
        h = GO.dequant_int(hq, qp.g[A.GRID["h"]], bool(qp.use_pot2))
        _check_equal(f"gru int32 output dir{d}", got[..., d * H:(d + 1) * H], h)
        if d == 0:
            _check_equal("gru int-IO codes dir0", gq[..., :H], hq)
    return {"sequences": list(rows), "forward": "bit-exact (int32 carrier and int-IO codes)"}


def _gru_c5_leg(torch, steps: int, warmup: int):
    """c5: QuantGRU unidirectional QAT fwd+bwd,
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

    dt, p50, p95, kernels, roof = _timed_steps(torch, step, steps, warmup,
                                               _gru_kernel_work(B, T, I, H, D=1,
                                                                stepped_bwd=True),
                                               traffic_prefix="c5_")
    _log(f"gru c5: {dt*1e3:.2f} ms/step wall, P50 {p50:.2f} ms, {B/dt:.1f} seq/s")
    for k, v in sorted(kernels.items(), key=lambda kv: -kv[1]["ms_per_step"]):
        _log(f"  {k}: {v['ms_per_step']:.3f} ms/step, {v['us_per_launch']:.1f} us/launch")
    return {"ms_per_step": dt * 1e3, "p50_ms": p50, "p95_ms": p95, "seq_per_s": B / dt,
            "kernels_ms_per_step": {k: round(v["ms_per_step"], 4) for k, v in kernels.items()},
            "roofline": roof}, m, x


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
        "lstm_bwd_weight_gemms": (2.0 * M * C * (2 * I + H), BF16_MFMA_PEAK,
                                  "dx, dW_ih, dW_hh GEMMs (float gradient split into three "
                                  "bf16 terms against exact bf16 code planes, MFMA)"),
        "lstm_fwd_input_gemm": (2.0 * M * C * I, INT8_MFMA_PEAK,
                                "input linear W_ih_q.x_q exact integer GEMM"),
    }


def _timed_steps(torch, step, steps, warmup, work, timed=None, traffic_prefix=""):
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
    if timed is None:
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
            "unit": "TFLOP/s", "frac": round(achieved / peak, 6),
            "traffic": _traffic(traffic_prefix + dom),
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


# The reference's only published numbers for this path: QuantLSTM CUDA FP32 q-carrier forward
# inference, timed from input quantisation to the dequantised final state with the static
# parameters cached (operators/quant-lstm/docs/cuda-performance.md:45-50; profiles and floors in
# tests/benchmarks/config/cuda_performance_thresholds_v1.json:24-58), on an NVIDIA RTX 6000D:
# (case id of the reference's strict matrix, profile, P50 ms, P95 ms, seq/s).
PUBLISHED_LSTM = [
    ("stage4_basic_cuda_fp32_pedantic_int8_bias_time", "cuda_gru_basic / pedantic",
     1.283040, 1.290176, 49882),
    ("stage4_basic_cuda_fp32_tf32_int16_no_bias_batch", "cuda_gru_basic / tf32",
     1.036768, 1.039744, 61730),
    ("stage4_performance_cuda_fp32_large_batch_pedantic", "large_batch / pedantic",
     0.416640, 0.419936, 307220),
    ("stage4_performance_cuda_fp32_large_batch_tf32", "large_batch / tf32",
     0.324608, 0.333952, 394322),
]


def _lstm_published_leg(torch, iters: int = 200, warmup: int = 20):
    """The reference's published QuantLSTM inference profiles: each case's resolved operator
    config (tests/golden/lstm/strict_matrix_cuda_cases.json, the reference's strict matrix) on
    its shape [T, B, I, H], calibrated on synthetic U(-1, 1) input, then the quantised forward
    (no checkpoints) called through the C ABI on time-major device buffers, as the reference's
    benchmark calls its C++ core.  Per-call hipEvents on the launch stream, P50 / P95 over
    ``iters`` calls after ``warmup``; seq/s = B / P50.  The weights are quantised inside every
    timed call (the reference caches them: its timed region is smaller).  Every case runs the
    exact arithmetic: its tf32 rows are the reference's faster, approximate math mode."""
    import ctypes

    import lstm_ops
    import quant_lstm as QL
    import rxmet_lib

    dev = torch.device("cuda:0")
    doc = json.loads((ROOT / "tests" / "golden" / "lstm" / "strict_matrix_cuda_cases.json").read_text())
    cases = {c["case_id"]: c for c in doc["cases"]}
    lib = rxmet_lib.load()
    stream = torch.cuda.current_stream(dev)
    out = {}
    for case_id, profile, ref_p50, ref_p95, ref_sps in PUBLISHED_LSTM:
        c = cases[case_id]
        T, B, I, H = c["shape"]
        bias = c["bias_profile"] != "disabled"
        torch.manual_seed(doc["parameter_seeds"][c["shape_profile"]])
        m = QL.QuantLSTM(I, H, bias=bias, quant_config=c["resolved_quant_config"]).to(dev)
        g = torch.Generator().manual_seed(1001)
        x = (torch.rand((T, B, I), generator=g) * 2 - 1).to(dev)
        m.calibrating = True
        with torch.no_grad():
            m(x)
        m.calibrating = False
        m.finalize_calibration()
        m.use_quantization = True
        m.eval()
        Wi, Wh, bi, bh = m._direction_params(False)
        prm = m._params[0].struct
        y = torch.empty((T, B, H), device=dev)
        hn = torch.empty((B, H), device=dev)
        cn = torch.empty((B, H), device=dev)
        ws = torch.empty(int(lib.rxmet_lstm_forward_workspace_bytes(T, B, I, H)), dtype=torch.uint8,
                         device=dev)
        ptr = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
        args = (T, B, I, H, ptr(Wi), ptr(Wh), ptr(bi), ptr(bh), ptr(x), None, None,
                ctypes.byref(prm), ptr(y), ptr(hn), ptr(cn), None, ptr(ws),
                ctypes.c_void_p(stream.cuda_stream))

        def call():
            rxmet_lib.call("rxmet_lstm_forward_quant", *args)

        with torch.no_grad():
            ref_out, _ = m(x)
        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        if not torch.equal(y, ref_out):
            raise ValidationError(f"lstm published {case_id}: C-ABI forward differs from the module")
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(iters + 1)]
        evs[0].record(stream)
        h0 = time.perf_counter()
        for i in range(iters):
            call()
            evs[i + 1].record(stream)
        host_ms = (time.perf_counter() - h0) / iters * 1e3
        torch.cuda.synchronize()
        per = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(iters))
        p50, p95 = per[len(per) // 2], per[min(len(per) - 1, int(0.95 * len(per)))]
        out[case_id] = {"profile": profile, "shape_TBIH": [T, B, I, H],
                        "bits": c["bitwidth_profile"], "p50_ms": round(p50, 4),
                        "p95_ms": round(p95, 4), "seq_per_s": round(B / (p50 * 1e-3), 1),
                        "reference_p50_ms": ref_p50, "reference_p95_ms": ref_p95,
                        "reference_seq_per_s": ref_sps,
                        "speedup_p50": round(ref_p50 / p50, 3),
                        "host_ms_per_call": round(host_ms, 4)}
        _log(f"lstm published {profile} {c['shape']}: P50 {p50:.4f} ms P95 {p95:.4f} ms "
             f"{B / (p50 * 1e-3):.0f} seq/s (reference RTX 6000D {ref_sps} seq/s); host "
             f"{host_ms:.4f} ms per call")
    return out


def _validate_lstm(torch, m, x, g, rows):
    """One more step of the benchmarked module: outputs and every gradient finite, the sampled
    sequences' output (bit-exact) and dx (1e-4) equal to the oracle's."""
    import numpy as np

    import lstm_oracle as LO

    m.zero_grad(set_to_none=True)
    xl = x.detach().clone().requires_grad_(True)
    out, _ = m(xl)
    out.backward(g)
    torch.cuda.synchronize()
    if not bool(torch.isfinite(out).all()) or not bool(torch.isfinite(xl.grad).all()):
        raise ValidationError("lstm: non-finite output or input gradient")
    for name, p in m.named_parameters():
        if not bool(torch.isfinite(p.grad).all()):
            raise ValidationError(f"lstm: non-finite gradient of {name}")
    Wi, Wh, bi, bh = (p.detach().cpu().numpy() for p in m._direction_params(False))
    prm = m._params[0].struct
    xs = x[:, rows].detach().contiguous().cpu().numpy()
    o = LO.forward_quant(Wi, Wh, bi, bh, xs, prm, mode=LO.ACT_LIBM_EXACT)
    _check_equal("lstm output", out[:, rows].detach().cpu().numpy(), o["output"])
    gr = LO.backward_quant(o, prm, g[:, rows].detach().contiguous().cpu().numpy())
    err = _check_close("lstm dx", xl.grad[:, rows].cpu().numpy(), gr["dx"])
    return {"sequences": list(rows), "forward": "bit-exact", "dx_max_abs_err_rel": err,
            "grads_finite": True}


def _timed_cpu(fn, budget_s: float):
    """Run fn until about budget_s seconds have passed (at least once); seconds per call."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            return dt / reps, reps


def _gru_cpu_baseline(m, x, rows: int, batch_first: bool, what: str, budget_s: float = 12.0):
    """The reference's own CPU PTQ forward (quantGRUForwardCPU, integer carrier; src/
    gru_host.cc:161-252, gru_forward_cpu_quant.cc), compiled from its sources into
    oracle/_ref, over every direction of the first `rows` sequences, with the module's
    calibrated ranges and bit-width configuration.  The reference has no CPU QAT
    (quant_gru.py:2171-2173), so this is forward only.  Without oracle/_ref: the C oracle's
    FP-carrier QAT forward+backward (kind "port")."""
    import numpy as np

    import gru_oracle as GO

    xt = x.detach().transpose(0, 1) if batch_first else x.detach()
    xs = xt[:, :rows].contiguous().cpu().numpy()
    T, Bs, I = xs.shape
    H = m.hidden_size
    dirs = _gru_dirs_haste(m)
    if GO.has_ref():
        def run():
            for d, (W, R, bw, br, _, rg, cfg) in enumerate(dirs):
                GO.ref_forward_ptq(W, R, bw, br, np.ascontiguousarray(xs[::-1]) if d else xs, rg,
                                   cfg)
        dt, reps = _timed_cpu(run, budget_s)
        return {"value": round(Bs / dt, 3), "unit": "seq/s", "cores": 1, "kind": "reference",
                "sample": f"{what}: the reference's quantGRUForwardCPU (integer-carrier PTQ "
                          f"forward, {len(dirs)} direction(s)) on {Bs} sequences (T={T}, I={I}, "
                          f"H={H}), one thread, {reps} run(s) of {dt:.2f} s; forward only: "
                          f"the reference has no CPU QAT",
                **_host_info()}
    dh = np.zeros((T + 1, Bs, H), np.float32)
    dh[1:] = 1e-6

    def run_port():
        for d, (W, R, bw, br, qp, _, _) in enumerate(dirs):
            fwd = GO.forward_quant(W, R, bw, br, np.ascontiguousarray(xs[::-1]) if d else xs, qp,
                                   training=True)
            GO.backward_quant(fwd, dh, qp)
    dt, reps = _timed_cpu(run_port, budget_s)
    return {"value": round(Bs / dt, 3), "unit": "seq/s", "cores": 1, "kind": "port",
            "sample": f"{what}: C oracle QAT forward+backward on {Bs} sequences, one thread",
            **_host_info()}


def _lstm_cpu_baseline(m, x, rows: int = 16, budget_s: float = 12.0):
    """The reference's own CPU q-carrier forward (lstmForwardQuantizedFpCpuReference,
    src/lstm/forward_quantized_fp_cpu.cc, compiled into oracle/_ref) on the first `rows`
    sequences of c4 with the module's grids; forward only (no CPU QAT in the reference,
    quant_lstm.py:751-756).  Without oracle/_ref: the C oracle's forward+backward."""
    import numpy as np

    import lstm_oracle as LO

    xs = x[:, :rows].detach().contiguous().cpu().numpy()
    Wi, Wh, bi, bh = (p.detach().cpu().numpy() for p in m._direction_params(False))
    prm = m._params[0].struct
    T, Bs, I = xs.shape
    if LO.has_ref():
        dt, reps = _timed_cpu(lambda: LO.ref_forward_fp(Wi, Wh, bi, bh, xs, prm), budget_s)
        return {"value": round(Bs / dt, 3), "unit": "seq/s", "cores": 1, "kind": "reference",
                "sample": f"c4: the reference's lstmForwardQuantizedFpCpuReference (q-carrier "
                          f"forward) on {Bs} of the 512 sequences (T={T}, I={I}, "
                          f"H={m.hidden_size}), one thread, {reps} run(s) of {dt:.2f} s; forward "
                          f"only: the reference has no CPU QAT",
                **_host_info()}
    g = np.full((T, Bs, m.hidden_size), 1e-3, np.float32)

    def run_port():
        LO.backward_quant(LO.forward_quant(Wi, Wh, bi, bh, xs, prm, mode=LO.ACT_LIBM), prm, g)
    dt, reps = _timed_cpu(run_port, budget_s)
    return {"value": round(Bs / dt, 3), "unit": "seq/s", "cores": 1, "kind": "port",
            "sample": f"c4: C oracle QAT forward+backward on {Bs} sequences, one thread",
            **_host_info()}


def _qdq_cpu_baseline(torch, budget_s: float = 8.0):
    """The reference's QDQ step on the host, as aten on CPU tensors with every intra-op thread:
    the learnable-encoding QuantDequantFunc forward+backward (torch_builtins.py:640-691)
    restated as aten operations, on the full c2 tensor [8192, 8192]; the frozen path
    (fake_quantize_per_tensor_affine forward + its STE backward, :287-361) reported beside it.
    GB/s on c2's byte formula (20 bytes per element, fwd+bwd)."""
    import qdq_oracle as O

    R = Cc = 8192
    torch.manual_seed(2)
    x = torch.randn(R, Cc)
    torch.manual_seed(5)
    g = torch.randn(R, Cc)
    s = torch.tensor(0.05)
    o = torch.tensor(-3.0)
    threads = torch.get_num_threads()
    dt, reps = _timed_cpu(lambda: O.torch_learnable_step(torch, x, g, s, o, -128, 127), budget_s)
    dtf, repsf = _timed_cpu(lambda: O.torch_frozen_step(torch, x, g, 0.05, 3, -128, 127),
                            budget_s / 2)
    n = R * Cc
    return {"value": round(20 * n / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"c2 per-tensor 8-bit learnable QDQ fwd+bwd on the full [{R}, {Cc}] tensor, "
                      f"aten on CPU ({threads} threads), {reps} run(s) of {dt:.3f} s",
            "frozen_fake_quantize_GB_s": round(20 * n / dtf / 1e9, 3),
            "frozen_note": "the reference's own frozen-encoding path (aten "
                           "fake_quantize_per_tensor_affine), same tensor and threads",
            "qc_op_one_shot": _qc_ref_cpu_baseline(x[:1024].contiguous().numpy(), budget_s / 2),
            **_host_info()}


def _qc_ref_cpu_baseline(xs, budget_s: float):
    """QcQuantizeOp's one-shot work on the reference's own CPU code (oracle/_ref/libqc_ref.so:
    MinMaxEncodingAnalyzer statistics + getComputedEncodings, then quantizeDequantizeBroadcast;
    one thread, as the reference runs them), 8-bit encodings per row of a [1024, 8192] slice of
    c2; GB/s on the GPU leg's byte formula (12 bytes per element).  None where the reference
    checker was not built."""
    import ctypes

    import numpy as np

    path = ROOT / "oracle" / "_ref" / "libqc_ref.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    R, Cc = xs.shape
    ts = np.array([R, Cc], np.int64)
    es = np.array([R, 1], np.int64)
    enc = np.zeros(4 * R, np.float64)
    y = np.empty_like(xs)
    P = ctypes.c_void_p

    def run():
        lib.qcref_analyzer(P(xs.ctypes.data), P(ts.ctypes.data), 2, P(es.ctypes.data), 2, 1, 8,
                           0, 0, 0, P(enc.ctypes.data))
        lib.qcref_qdq(P(xs.ctypes.data), P(y.ctypes.data), P(ts.ctypes.data), 2,
                      P(es.ctypes.data), 2, P(enc.ctypes.data), 8)
    dt, reps = _timed_cpu(run, budget_s)
    return {"value": round(12 * xs.size / dt / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "reference",
            "sample": f"QcQuantizeOp oneShot, 8-bit per-row encodings, [{R}, {Cc}] slice of c2, "
                      f"{reps} run(s) of {dt:.3f} s"}


FP32_MFMA_PEAK = 157.3


def _calib_leg(torch, steps: int, warmup: int):
    """calib: the MinMax calibration forwards (float recurrence plus the statistics of every
    grid, rxmet_gru_forward_calibrate / rxmet_lstm_forward_calibrate) at the benchmark shapes:
    c3 GRU (bidirectional, both directions per step), c4 LSTM and c5 GRU.  One step = one
    calibration forward over the whole batch, merged into the module's running ranges as a
    calibration loop over batches does."""
    import quant_gru as QG
    import quant_lstm as QL

    dev = torch.device("cuda:0")
    res, keep = {}, {}
    cases = (("gru_c3", "gru", 256, 200, 80, 256, True),
             ("lstm_c4", "lstm", 512, 100, 64, 512, False),
             ("gru_c5", "gru", 1024, 50, 256, 1024, False))
    for name, kind, B, T, I, H, bidir in cases:
        torch.manual_seed(6)
        if kind == "gru":
            x = torch.randn(T, B, I)
            m = QG.QuantGRU(I, H, bidirectional=bidir)
            C = 3 * H
        else:
            x = torch.rand(T, B, I) * 2 - 1
            m = QL.QuantLSTM(I, H)
            C = 4 * H
        m = m.to(dev)
        x = x.to(dev)
        D = 2 if bidir else 1

        def step(m=m, x=x):
            m.calibrating = True
            with torch.no_grad():
                m(x)
            m.calibrating = False

        M = T * B
        rec, gemm = f"{kind}_calibrate_forward", f"{kind}_calibrate_input_gemm"
        work = {rec: (D * 2.0 * M * H * C, FP32_MFMA_PEAK,
                      "recurrent GEMM h R of every direction over T steps on fp32 MFMA (one "
                      "clustered launch per direction: gates and statistics fused)"),
                gemm: (D * 2.0 * M * C * I, FP32_MFMA_PEAK,
                       "input projection x W of every direction (fp32 MFMA, statistics fused)")}
        dt, p50, p95, kernels, roof = _timed_steps(torch, step, steps, warmup, work,
                                                   timed=[rec], traffic_prefix=f"{name}_")
        _log(f"calibration {name}: {dt*1e3:.3f} ms/step wall, P50 {p50:.3f} ms, {B/dt:.1f} "
             f"seq/s; " + ", ".join(f"{k} {v['ms_per_step']:.3f} ms/step"
                                    for k, v in kernels.items()))
        res[name] = {"ms_per_step": dt * 1e3, "p50_ms": p50, "p95_ms": p95, "seq_per_s": B / dt,
                     "shape_TBIH": [T, B, I, H], "directions": D,
                     "kernels_ms_per_step": {k: round(v["ms_per_step"], 4)
                                             for k, v in kernels.items()},
                     "recurrence_roofline": {k: roof[k] for k in ("achieved", "peak", "unit",
                                                                  "frac", "us_per_launch",
                                                                  "traffic")}}
        keep[name] = (kind, m, x)
    return res, keep


def _validate_calib(torch, keep, rows=(0, -1)):
    """One more calibration forward of each benchmarked module: every output finite, the
    input range equal to the tensor's own min / max, and the sampled sequences' output equal
    to the oracle's float calibration forward run on those sequences alone (rtol 1e-4)."""
    import numpy as np

    import gru_oracle as GO
    import lstm_oracle as LO
    import rxmet_lstm_abi as L

    out = {}
    for name, (kind, m, x) in keep.items():
        m.calibrating = True
        with torch.no_grad():
            y = m(x)[0]
        m.calibrating = False
        torch.cuda.synchronize()
        if not bool(torch.isfinite(y).all()):
            raise ValidationError(f"{name} calibration: non-finite output")
        B = x.shape[1]
        rws = sorted({r % B for r in rows})
        xs = x[:, rws].contiguous().cpu().numpy()
        got = y[:, rws].cpu().numpy()
        H = m.hidden_size
        err = 0.0
        if kind == "gru":
            lo, hi = float(x.min()), float(x.max())
            rg = m.quant_ranges
            if rg.min_x_ != lo or rg.max_x_ != hi:
                raise ValidationError(f"{name} calibration: x range [{rg.min_x_}, {rg.max_x_}] "
                                      f"is not the input's [{lo}, {hi}]")
            for d in range(m.num_directions):
                sfx = "_reverse" if d else ""
                p = lambda n: getattr(m, n + sfx).detach().cpu().numpy()
                W = np.ascontiguousarray(_swap_gates(p("weight_ih_l0")).T)
                R = np.ascontiguousarray(_swap_gates(p("weight_hh_l0")).T)
                bw, br = _swap_gates(p("bias_ih_l0")), _swap_gates(p("bias_hh_l0"))
                xd = np.ascontiguousarray(xs[::-1]) if d else xs
                h, _, _ = GO.forward_calibrate(W, R, bw, br, xd)
                exp = h[1:][::-1] if d else h[1:]
                err = max(err, _check_close(f"{name} calibration output (direction {d})",
                                            got[..., d * H:(d + 1) * H], exp))
        else:
            lo, hi = float(x.min()), float(x.max())
            st = m._stats[0].cpu().numpy()
            n = L.NOPS  # minima of the operators, then maxima; "input" first
            if float(st[0]) != lo or float(st[n]) != hi:
                raise ValidationError(f"{name} calibration: input range [{st[0]}, {st[n]}] is "
                                      f"not the input's [{lo}, {hi}]")
            Wi, Wh, bi, bh = (p.detach().cpu().numpy() for p in m._direction_params(False))
            exp, _, _ = LO.forward_float(Wi, Wh, bi, bh, xs, mode=LO.ACT_CR)
            err = _check_close(f"{name} calibration output", got, exp)
        out[name] = {"sequences": rws,
                     "output_vs_oracle": f"rtol 1e-4; max |err| / max |ref| = {err:.3g}",
                     "input_range": "exact"}
    return out


def _c1_leg(torch, steps: int, warmup: int):
    """c1: the PTQ calibration pass of a unidirectional QuantGRU (B=32, T=98, I=40, H=64):
    MinMax calibration forward on the GPU, parameter derivation, then the PTQ (quantised,
    eval) forward.  One step = that whole pass over the batch."""
    import quant_gru as QG
    import rxmet_gru_abi as A

    dev = torch.device("cuda:0")
    B, T, I, H = 32, 98, 40, 64
    torch.manual_seed(1)
    x = torch.randn(B, T, I)
    m = QG.QuantGRU(I, H, batch_first=True)
    torch.nn.init.xavier_uniform_(m.weight_ih_l0)
    torch.nn.init.xavier_uniform_(m.weight_hh_l0)
    m.set_all_bitwidth(8, is_symmetric=False)
    for k in ("W_granularity_", "R_granularity_", "bw_granularity_", "br_granularity_"):
        setattr(m._bitwidth_config, k, A.PER_TENSOR)
    m = m.to(dev).eval()
    x = x.to(dev)
    out = {}

    def step():
        with torch.no_grad():
            m.use_quantization = False
            with m.calibration_context():  # reset, MinMax forward, derive the grids
                m(x)
            m.use_quantization = True
            out["y"] = m(x)[0]

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    per = []
    for _ in range(steps):
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        per.append(time.perf_counter() - t0)
    dt = sum(per) / len(per)
    per.sort()
    # the same passes back to back (one synchronisation after the last): the host prepares the
    # next pass while the GPU runs this one, as a calibration loop over many batches does
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt_pipe = (time.perf_counter() - t0) / steps
    _log(f"gru c1: {dt*1e3:.3f} ms per calibration + PTQ pass (each pass synchronised), "
         f"{B/dt:.1f} seq/s; back to back {dt_pipe*1e3:.3f} ms")
    return {"ms_per_step": dt * 1e3, "p50_ms": per[len(per) // 2] * 1e3, "seq_per_s": B / dt,
            "back_to_back_ms_per_step": dt_pipe * 1e3}, m, x, out["y"]


def _validate_c1(m, x, y):
    """The GPU's PTQ output of every c1 sequence equals the oracle's FP-carrier forward with the
    module's grids, bit for bit."""
    import numpy as np

    import gru_oracle as GO

    W, R, bw, br, qp, _, _ = _gru_dirs_haste(m)[0]
    xs = x.detach().transpose(0, 1).contiguous().cpu().numpy()
    fwd = GO.forward_quant(W, R, bw, br, xs, qp, training=False)
    _check_equal("c1 PTQ output", y.transpose(0, 1).cpu().numpy(), fwd["h"][1:])
    return {"sequences": "all 32", "forward": "bit-exact"}


def _c1_cpu_baseline(m, x, budget_s: float = 10.0):
    """The reference's own CPU PTQ calibration pass on the whole c1 batch: forwardWithCalibrationCPU
    (src/gru_forward_cpu.cc:58-151), calculateGRUQuantitativeParameters (src/gru_host.cc:13-124)
    and the PTQ forward quantGRUForwardCPU (:161-252), compiled into oracle/_ref; one thread
    (the reference has no OpenMP there).  Without oracle/_ref: the C oracle's calibration and
    FP-carrier forward."""
    import numpy as np

    import gru_oracle as GO
    import rxmet_gru_abi as A

    W, R, bw, br, qp, _, cfg = _gru_dirs_haste(m)[0]
    xs = x.detach().transpose(0, 1).contiguous().cpu().numpy()
    T, B, I = xs.shape
    H = m.hidden_size
    ref = GO.has_ref()

    def run():
        _, _, stats = GO.forward_calibrate(W, R, bw, br, xs, ref=ref)
        ranges = A.make_ranges(stats, H)
        if ref:
            GO.ref_forward_ptq(W, R, bw, br, xs, ranges, cfg)
        else:
            q, _ = GO.make_params(ranges, cfg)
            GO.forward_quant(W, R, bw, br, xs, q, training=False)
    dt, reps = _timed_cpu(run, budget_s)
    return {"value": round(B / dt, 3), "unit": "seq/s", "cores": 1,
            "kind": "reference" if ref else "port",
            "sample": f"c1: {'the reference' if ref else 'C oracle'} calibration forward + "
                      f"parameter derivation + PTQ forward on all {B} sequences (T={T}, I={I}, "
                      f"H={H}), one thread, {reps} run(s) of {dt:.3f} s",
            **_host_info()}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-validate", action="store_true",
                    help="skip the oracle comparison of the benchmarked outputs (profiling runs)")
    ap.add_argument("--legs", default="gru,lstm,qdq,c1,c5,gint,lstmpub,calib",
                    help="comma-separated subset of gru,lstm,qdq,c1,c5,gint,lstmpub,calib")
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
    validate = not args.no_validate
    checks = {}
    gru = roof = lstm = lstm_roof = qdq = qdq_roof = c5 = c1 = gint = gint_roof = None
    lstmpub = calib = None
    try:
        if "gru" in legs:
            gru, roof, m, x = _gru_leg(torch, args.steps, args.warmup)
            if validate:
                checks["c3"] = _validate_gru(torch, m, x, [0, 255], batch_first=True)
                _log(f"c3 validation: {checks['c3']}")
        if "lstm" in legs:
            lstm, lstm_roof, lm, lx, lg = _lstm_leg(torch, args.steps, args.warmup)
            if validate:
                checks["c4"] = _validate_lstm(torch, lm, lx, lg, [0, 511])
                _log(f"c4 validation: {checks['c4']}")
        if "qdq" in legs:
            qdq, qdq_roof, qcheck = _qdq_leg(torch, args.steps, args.warmup, validate)
            if qcheck is not None:
                checks["c2"] = qcheck
        if "c1" in legs:
            c1, c1m, c1x, c1y = _c1_leg(torch, args.steps, args.warmup)
            if validate:
                checks["c1"] = _validate_c1(c1m, c1x, c1y)
        if "gint" in legs:
            gint, gint_roof, gm, gx, gout = _gru_int_leg(torch, args.steps, args.warmup)
            if validate:
                checks["gint"] = _validate_gru_int(gm, gx, gout["y"], gout["q"], [0, 255])
                _log(f"gint validation: {checks['gint']}")
        if "lstmpub" in legs:
            lstmpub = _lstm_published_leg(torch)
        if "calib" in legs:
            calib, ckeep = _calib_leg(torch, args.steps, args.warmup)
            if validate:
                checks["calibration"] = _validate_calib(torch, ckeep)
                _log(f"calibration validation: {checks['calibration']}")
            del ckeep
        if "c5" in legs:
            c5, c5m, c5x = _gru_c5_leg(torch, args.steps, args.warmup)
            if validate:
                checks["c5"] = _validate_gru(torch, c5m, c5x, [1023], batch_first=False)
                _log(f"c5 validation: {checks['c5']}")
    except ValidationError as e:
        print(f"bench.py: the benchmarked path failed its check: {e}", file=sys.stderr)
        return 3
    cpu = cpu_qdq = cpu_lstm = cpu_c1 = cpu_c5 = None
    if not args.no_cpu_baseline:
        if gru is not None:
            cpu = _gru_cpu_baseline(m, x, 32, True, "c3")
            _log(f"c3 cpu baseline: {cpu}")
        if lstm is not None:
            cpu_lstm = _lstm_cpu_baseline(lm, lx)
            _log(f"c4 cpu baseline: {cpu_lstm}")
        if qdq is not None:
            cpu_qdq = _qdq_cpu_baseline(torch)
            _log(f"c2 cpu baseline: {cpu_qdq}")
        if c1 is not None:
            cpu_c1 = _c1_cpu_baseline(c1m, c1x)
            _log(f"c1 cpu baseline: {cpu_c1}")
        if c5 is not None:
            cpu_c5 = _gru_cpu_baseline(c5m, c5x, 8, False, "c5", budget_s=8.0)
            _log(f"c5 cpu baseline: {cpu_c5}")
        if gint is not None and cpu is None:
            cpu = _gru_cpu_baseline(gm, gx, 32, True, "c3")
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
        "gru_c1": rnd(c1),
        "gru_c5": rnd(c5),
        "gru_int32_c3": rnd(gint),
        "gru_int32_roofline": gint_roof,
        "calibration_forward": calib,
        "lstm_published_inference": lstmpub,
        "qdq": None if qdq is None else {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                                             for kk, vv in v.items()} for k, v in qdq.items()},
        "roofline": roof,
        "lstm_roofline": lstm_roof,
        "qdq_roofline": qdq_roof,
        "cpu_baseline": cpu,
        "lstm_cpu_baseline": cpu_lstm,
        "qdq_cpu_baseline": cpu_qdq,
        "c1_cpu_baseline": cpu_c1,
        "c5_cpu_baseline": cpu_c5,
        "validation": checks if validate else None,
    }
    print(json.dumps(line), flush=True)
    _end_children()
    return 0


def _end_children() -> None:
    """End any child process this run left behind (none is started on purpose), so that the
    benchmark exits with nothing of its own still running."""
    try:
        import psutil
    except ImportError:
        return
    kids = psutil.Process().children(recursive=True)
    for k in kids:
        k.terminate()
    _, alive = psutil.wait_procs(kids, timeout=5)
    for k in alive:
        k.kill()
    if kids:
        _log(f"ended {len(kids)} leftover child process(es): {[k.pid for k in kids]}")


if __name__ == "__main__":
    sys.exit(main())
