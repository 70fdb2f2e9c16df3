"""Writes the known-answer fixtures, transcribed as data from the reference's
own tests:

* kat_cpu_convolution.json: the three known-answer tests of the scalar CPU
  convolution kernels, RiemannEngine tests/convolution/test_cpu_convolution.cpp
  :15-61 (inputs, maps and expected outputs; weights [k][cin][cout]).
* kat_layers_pooling.json: the pooling known answers of
  tests/engine/test_layers.cpp:26-115 (inputs and the expected value of each
  checked output row, keyed by its coordinate or batch).

Run: python tests/golden/make_golden.py
"""
import json
import os

KATS = [
    {   # test_cpu_convolution.cpp:15-26
        "name": "pointwise_forward_identity_mapping",
        "kind": "forward", "cin": 2, "cout": 2, "n_in": 3, "n_out": 3,
        "x": [1, 2, 3, 4, 5, 6], "weight": [1, 2, 3, 4],
        "in_maps": [[0, 1, 2]], "out_maps": [[0, 1, 2]],
        "expected_y": [7, 10, 15, 22, 23, 34],
    },
    {   # test_cpu_convolution.cpp:28-46
        "name": "pointwise_backward_identity_mapping",
        "kind": "backward", "cin": 2, "cout": 2, "n_in": 3, "n_out": 3,
        "x": [1, 2, 3, 4, 5, 6], "grad_y": [1, 2, 3, 4, 5, 6], "weight": [1, 2, 3, 4],
        "in_maps": [[0, 1, 2]], "out_maps": [[0, 1, 2]],
        "expected_grad_x": [5, 11, 11, 25, 17, 39],
        "expected_grad_w": [35, 44, 44, 56],
    },
    {   # test_cpu_convolution.cpp:48-61
        "name": "pointwise_forward_nonidentity_mapping",
        "kind": "forward", "cin": 1, "cout": 1, "n_in": 3, "n_out": 3,
        "x": [1, 3, 5], "weight": [2],
        "in_maps": [[2, 0, 1]], "out_maps": [[1, 2, 0]],
        "expected_y": [6, 10, 2],
    },
]

# test_layers.cpp:26-37 (make_two_batches) and :58-78
TWO_BATCHES = {
    "coords": [[0, 0, 0, 0], [0, 1, 0, 0], [1, 0, 0, 0], [1, 2, 2, 2]],
    "features": [[1.0, 2.0], [3.0, 4.0], [10.0, 20.0], [30.0, 40.0]],
}
GLOBAL_KATS = [
    {"mode": "avg", "batch": 0, "expected": [2.0, 3.0]},
    {"mode": "avg", "batch": 1, "expected": [20.0, 30.0]},
    {"mode": "max", "batch": 0, "expected": [3.0, 4.0]},
    {"mode": "sum", "batch": 1, "expected": [40.0, 60.0]},
]
# test_layers.cpp:80-115: kernel_size 2, stride 2
STRIDED = {
    "coords": [[0, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0], [0, 2, 0, 0], [0, 3, 1, 1]],
    "features": [[1.0], [2.0], [3.0], [10.0], [20.0]],
    "kernel_size": 2, "stride": 2, "out_rows": 2, "out_tensor_stride": [2, 2, 2],
}
STRIDED_KATS = [
    {"mode": "avg", "coordinate": [0, 0, 0], "expected": 2.0},
    {"mode": "avg", "coordinate": [2, 0, 0], "expected": 15.0},
    {"mode": "max", "coordinate": [0, 0, 0], "expected": 3.0},
    {"mode": "max", "coordinate": [2, 0, 0], "expected": 20.0},
    {"mode": "sum", "coordinate": [0, 0, 0], "expected": 6.0},
]


def write_pooling(folder):
    out = os.path.join(folder, "kat_layers_pooling.json")
    with open(out, "w") as f:
        json.dump({"source": "RiemannEngine tests/engine/test_layers.cpp:26-115",
                   "tolerance_abs": 1e-5,
                   "global": {"input": TWO_BATCHES, "kats": GLOBAL_KATS},
                   "strided": {"input": STRIDED, "kats": STRIDED_KATS}}, f, indent=1)
    print("wrote", out)


if __name__ == "__main__":
    write_pooling(os.path.dirname(os.path.abspath(__file__)))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kat_cpu_convolution.json")
    with open(out, "w") as f:
        json.dump({"source": "RiemannEngine tests/convolution/test_cpu_convolution.cpp:15-61",
                   "tolerance_abs": 1e-5, "kats": KATS}, f, indent=1)
    print("wrote", out)
