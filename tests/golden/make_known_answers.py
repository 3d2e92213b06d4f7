"""Writes reference_known_answers.json: the inputs and expected outputs that whisper4j's own unit tests
hold for the operations of the decoder step (paths relative to src/test/java/com/sparrowlogic/whisper4j/).
The values are transcribed from those tests' sources (read, not run: the reference needs a JDK this
image does not have); tests/test_oracle.py checks the oracle against every entry.

    python tests/golden/make_known_answers.py
"""

import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = {
    "dot": [
        {"cite": "tensor/SimdOpsTest.java:23-31", "a": [1, 2, 3, 4], "b": [5, 6, 7, 8], "expect": 70.0, "tol": 1e-4},
    ],
    # Linear takes W as [out][in]; the reference's matmul cases are restated as x @ W^T.
    "linear": [
        {"cite": "tensor/TensorTest.java:9-20", "x": [[1, 2, 3], [4, 5, 6]], "w": [[7, 9, 11], [8, 10, 12]],
         "expect": [[58, 64], [139, 154]], "tol": 1e-4},
        {"cite": "tensor/TensorTest.java:222-244", "x": [[1, 2], [3, 4]], "w": [[5, 6], [7, 8]],
         "expect": [[17, 23], [39, 53]], "tol": 1e-4},
        {"cite": "tensor/TensorTest.java:222-244", "x": [[1, 2, 3], [4, 5, 6]], "w": [[1, 2, 3], [4, 5, 6]],
         "expect": [[14, 32], [32, 77]], "tol": 1e-4},
        {"cite": "tensor/TensorTest.java:246-256", "x": [[1, 2, 3, 4]],
         "w": [[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0]], "expect": [[1, 2, 3]], "tol": 1e-4},
    ],
    "softmax": [
        {"cite": "tensor/TensorTest.java:270-278", "x": [[1, 2, 3, 4]], "expect": [[0.0321, 0.0871, 0.2369, 0.6439]],
         "tol": 1e-3},
    ],
    "softmax_row_sums": [
        {"cite": "tensor/TensorTest.java:78-85", "x": [[1, 2, 3], [10, 20, 30]], "expect": [1.0, 1.0], "tol": 1e-4},
    ],
    "layernorm": [
        {"cite": "tensor/TensorTest.java:280-290", "x": [[1, 2, 3, 4, 5]], "gamma": [1, 1, 1, 1, 1],
         "beta": [0, 0, 0, 0, 0], "columns": [0, 2, 4], "expect": [[-1.4142, 0.0, 1.4142]], "tol": 1e-3},
        {"cite": "tensor/TensorTest.java:99-106", "x": [[0, 0, 0, 0]], "gamma": [2, 2, 2, 2], "beta": [1, 1, 1, 1],
         "columns": [0, 1, 2, 3], "expect": [[1.0, 1.0, 1.0, 1.0]], "tol": 1e-4},
    ],
    "layernorm_row_mean": [
        {"cite": "tensor/TensorTest.java:88-97", "x": [[1, 2, 3, 4]], "gamma": [1, 1, 1, 1], "beta": [0, 0, 0, 0],
         "expect": [0.0], "tol": 1e-4},
    ],
    "gelu": [
        {"cite": "tensor/TensorTest.java:292-301", "x": [-2, -1, 0, 1, 2],
         "expect": [-0.0454, -0.1588, 0.0, 0.8412, 1.9546], "tol": 0.01},
        {"cite": "tensor/TensorTest.java:42-46", "x": [0.0], "expect": [0.0], "tol": 1e-5},
        {"cite": "tensor/TensorTest.java:54-58", "x": [-3.0], "expect": [0.0], "tol": 0.01},
    ],
}

if __name__ == "__main__":
    out = {"source": "whisper4j unit tests, src/test/java/com/sparrowlogic/whisper4j/ (file:line per case)", **CASES}
    with open(os.path.join(HERE, "reference_known_answers.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
