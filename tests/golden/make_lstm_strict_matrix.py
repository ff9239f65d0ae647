"""Writes tests/golden/lstm/strict_matrix_cuda_cases.json: the CUDA FP32 q-carrier cases of the
reference's strict precision matrix (operators/quant-lstm/tests/precision/config/
strict_matrix_v2.json), reduced to what the GPU parity test uses — case id, shape [T, B, I, H],
bias, layout and state profiles, the resolved quant config — plus the parameter seeds of
synthetic_data.json.  Data only; run in a checkout that has /root/reference."""
import json
from pathlib import Path

REF = Path("/root/reference/operators/quant-lstm/tests/precision/config")
OUT = Path(__file__).resolve().parent / "lstm" / "strict_matrix_cuda_cases.json"


def main():
    matrix = json.loads((REF / "strict_matrix_v2.json").read_text())
    synth = json.loads((REF / "synthetic_data.json").read_text())
    keep = ("case_id", "shape_profile", "shape", "state_profile", "bias_profile", "layout_profile",
            "batch_first", "bitwidth_profile", "resolved_quant_config")
    cases = [{k: c[k] for k in keep} for c in matrix["cases"] if c["backend"] == "cuda_fp32"]
    doc = {"source": "operators/quant-lstm/tests/precision/config/strict_matrix_v2.json "
                     "(cuda_fp32 cases), synthetic_data.json (parameter seeds)",
           "matrix_version": matrix["matrix_version"],
           "parameter_seeds": synth["parameter_seeds"], "cases": cases}
    OUT.write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {len(cases)} cases to {OUT}")


if __name__ == "__main__":
    main()
