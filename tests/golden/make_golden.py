"""Writes kat_cpu_convolution.json: the three known-answer tests of the
reference's scalar CPU convolution kernels, transcribed as data from
RiemannEngine tests/convolution/test_cpu_convolution.cpp:15-61
(inputs, maps and expected outputs; channel-major weights [k][cin][cout]).

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

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kat_cpu_convolution.json")
    with open(out, "w") as f:
        json.dump({"source": "RiemannEngine tests/convolution/test_cpu_convolution.cpp:15-61",
                   "tolerance_abs": 1e-5, "kats": KATS}, f, indent=1)
    print("wrote", out)
