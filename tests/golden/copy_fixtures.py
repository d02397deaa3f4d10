"""Copies the reference's operator fixtures for the quantized-weight path into tests/golden/ops.

Each fixture directory of the reference (test/fixtures/ops/<case>) holds one single-node ONNX
graph (model.onnx), its inputs (in_*.bin), the ONNX Runtime outputs (out_*.bin, raw little
endian) and meta.json. They were written by the reference's test/support/make_op_fixtures.py
(:136-196 quantization, :1109-1187 and :1486-1504 QMoE, :1434-1451 exact integer sums,
:1584-1594 large blocks) with ONNX Runtime CPU and graph optimisations off. They are data:
inputs and expected outputs, copied byte for byte.

Usage: python tests/golden/copy_fixtures.py [/root/reference]
"""

import os
import shutil
import sys

CASES = [
    "MatMulNBits_b2_bs16_packed",
    "MatMulNBits_b4_bs16_float",
    "MatMulNBits_b4_bs16_packed",
    "MatMulNBits_b4_bs256_packed",
    "MatMulNBits_b4_bs32_none_bias",
    "MatMulNBits_b8_bs32_packed",
    "GatherBlockQuantized_b4",
    "GatherBlockQuantized_b8",
    "DequantizeLinear_blocked",
    "DequantizeLinear_int32_f16_scale",
    "DequantizeLinear_per_axis",
    "DequantizeLinear_per_tensor",
    "MatMulInteger",
    "MatMulInteger_dynamic_quant",
    "MatMulInteger_k4096_extremes",
    "MatMulInteger_k4096_signed",
    "DynamicQuantizeLinear",
    "DynamicQuantizeLinear_all_zeros",
    "DynamicQuantizeLinear_ties",
    "QMoE_4bit_per_row_zero_points",
    "QMoE_4bit_silu_k2",
    "QMoE_4bit_silu_k2_decode",
    "QMoE_4bit_swiglu_k2_normalize",
    "QMoE_8bit_per_row_zero_points",
    "QMoE_8bit_silu_k1",
]


def main():
    reference = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    src_root = os.path.join(reference, "test", "fixtures", "ops")
    dst_root = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ops")
    os.makedirs(dst_root, exist_ok=True)
    for case in CASES:
        src = os.path.join(src_root, case)
        dst = os.path.join(dst_root, case)
        if os.path.isdir(dst):
            shutil.rmtree(dst)
        os.makedirs(dst)
        for name in sorted(os.listdir(src)):
            shutil.copyfile(os.path.join(src, name), os.path.join(dst, name))
            os.chmod(os.path.join(dst, name), 0o644)
        print("copied", case)


if __name__ == "__main__":
    main()
