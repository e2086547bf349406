"""Writes tests/golden/reference_known_answers.json.

The reference holds no golden files; its hot-path tests pin results with
closed-form known answers. This script transcribes those inputs and expected
outputs (data only) into one fixture, each with the reference test it comes
from. Element-wise ReLU / leaky-ReLU / bias cases are expressed through the
dense path with an identity W (X @ I is exact), which is how the HIP
runtime exposes them.

Run from the repository root:  python tests/golden/make_known_answers.py
"""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f32(a):
    return np.asarray(a, dtype=np.float32)


def case(name, src, pattern, dtype, inputs, expected, rtol=0.0, atol=0.0, alpha=0.01):
    return {"name": name, "source": src, "pattern": pattern, "dtype": dtype,
            "inputs": [np.asarray(x).tolist() for x in inputs],
            "expected": np.asarray(expected).tolist(), "rtol": rtol, "atol": atol,
            "alpha": alpha}


def main():
    I2, I4 = np.eye(2, dtype=np.float32), np.eye(4, dtype=np.float32)
    A = f32([[1, 2], [3, 4]])
    cases = [
        case("matmul_identity", "tests/linalg/test_matmul_execution.py:20-30", "matmul", "f32",
             [A, I2], A, rtol=1e-4),
        case("matmul_known_2x2", "tests/linalg/test_matmul_execution.py:32-42", "matmul", "f32",
             [A, f32([[5, 6], [7, 8]])], f32([[19, 22], [43, 50]]), rtol=1e-3),
        case("matmul_ones_8x8", "tests/linalg/test_matmul_execution.py:44-54", "matmul", "f32",
             [np.ones((8, 8), np.float32)] * 2, np.full((8, 8), 8.0, np.float32), atol=1e-5),
        case("matmul_ones_16x16", "tests/linalg/test_matmul_execution.py:56-66", "matmul", "f32",
             [np.ones((16, 16), np.float32)] * 2, np.full((16, 16), 16.0, np.float32), atol=1e-4),
        case("matmul_zeros", "tests/linalg/test_matmul_execution.py:81-91", "matmul", "f32",
             [A, np.zeros((2, 2), np.float32)], np.zeros((2, 2), np.float32), atol=1e-5),
        case("matmul_integer_identity", "tests/linalg/test_matmul_execution.py:93-103", "matmul",
             "i32", [np.eye(2, dtype=np.int32), np.array([[5, 6], [7, 8]], np.int32)],
             np.array([[5, 6], [7, 8]], np.int32)),
        case("matmul_rectangular_ones", "tests/linalg/test_binary_op_execution.py:176-186",
             "matmul", "f32", [np.ones((2, 3), np.float32), np.ones((3, 4), np.float32)],
             np.full((2, 4), 3.0, np.float32), rtol=1e-5),
        case("dense_layer_no_activation", "tests/linalg/test_binary_op_execution.py:193-206",
             "matmul_bias", "f32",
             [f32([[1, 0, 0, 0], [0, 1, 0, 0]]), np.ones((4, 3), np.float32), f32([0.1, 0.2, 0.3])],
             f32([[1, 0, 0, 0], [0, 1, 0, 0]]) @ np.ones((4, 3), np.float32) + f32([0.1, 0.2, 0.3]),
             rtol=1e-4),
        case("bias_add_2x4", "tests/linalg/test_binary_op_execution.py:114-124", "matmul_bias",
             "f32", [f32([[1, 2, 3, 4], [5, 6, 7, 8]]), I4, f32([0.1, 0.2, 0.3, 0.4])],
             f32([[1, 2, 3, 4], [5, 6, 7, 8]]) + f32([0.1, 0.2, 0.3, 0.4]), rtol=1e-5),
        case("bias_add_zeros_identity", "tests/linalg/test_binary_op_execution.py:137-146",
             "matmul_bias", "f32",
             [np.arange(9, dtype=np.float32).reshape(3, 3), np.eye(3, dtype=np.float32),
              np.zeros(3, np.float32)], np.arange(9, dtype=np.float32).reshape(3, 3), rtol=1e-5),
        case("relu_mixed", "tests/linalg/test_map_execution.py:74-82", "matmul_relu", "f32",
             [f32([[-1, 2, -3, 4]]), I4], f32([[0, 2, 0, 4]]), atol=1e-5),
        case("relu_all_negative", "tests/linalg/test_map_execution.py:64-72", "matmul_relu", "f32",
             [f32([[-1, -2, -3, -4]]), I4], f32([[0, 0, 0, 0]]), atol=1e-5),
        case("relu_all_positive", "tests/linalg/test_map_execution.py:54-62", "matmul_relu", "f32",
             [f32([[1, 2, 3, 4]]), I4], f32([[1, 2, 3, 4]]), atol=1e-5),
        case("manual_relu_if", "tests/linalg/test_map_execution.py:40-52", "matmul_relu", "f32",
             [f32([[-1, 0, 2, -3]]), I4], f32([[0, 0, 2, 0]]), atol=1e-5),
        case("relu_2d_mixed", "tests/linalg/test_map_execution.py:120-129", "matmul_relu", "f32",
             [f32([[-1, 2, -3, 4], [5, -6, 7, -8]]), I4],
             np.maximum(f32([[-1, 2, -3, 4], [5, -6, 7, -8]]), 0), rtol=1e-5),
        case("leaky_relu_negative_scaling", "tests/linalg/test_map_execution.py:94-103",
             "dense_leaky", "f32", [f32([[-1, -2, -10, -0.5]]), I4, np.zeros(4, np.float32)],
             f32([[-0.1, -0.2, -1.0, -0.05]]), atol=1e-5, alpha=0.1),
        case("leaky_relu_positive_passthrough", "tests/linalg/test_map_execution.py:84-92",
             "dense_leaky", "f32", [f32([[1, 2, 3, 4]]), I4, np.zeros(4, np.float32)],
             f32([[1, 2, 3, 4]]), atol=1e-5, alpha=0.1),
        case("leaky_relu_2d", "tests/linalg/test_map_execution.py:151-162", "dense_leaky", "f32",
             [f32([[-1, 2, -3, 4], [5, -6, 7, -8]]), I4, np.zeros(4, np.float32)],
             np.where(f32([[-1, 2, -3, 4], [5, -6, 7, -8]]) > 0,
                      f32([[-1, 2, -3, 4], [5, -6, 7, -8]]),
                      f32([[-1, 2, -3, 4], [5, -6, 7, -8]]) * np.float32(0.1)), rtol=1e-4,
             alpha=0.1),
    ]
    with open(os.path.join(HERE, "reference_known_answers.json"), "w") as f:
        json.dump({"note": "transcribed known answers from the reference's hot-path tests",
                   "cases": cases}, f, indent=1)
    print(f"{len(cases)} cases")


if __name__ == "__main__":
    main()
