"""Writes reference_kats.json: the expected values that the reference's own
tests assert for the hot path (closed-form known answers).  The numbers are
taken from the cited test files of gifton/VectorStoreKit
(Tests/VectorStoreKitTests/...); nothing of the reference is imported or run.

    python tests/golden/make_kats.py
"""
import json
import math
import os

KATS = {
    "source": "Tests/VectorStoreKitTests of gifton/VectorStoreKit",
    "vector512": {
        "_cite": "Vector512Tests.swift:61-67 (dot 1*2*512), :69-78 (512*(3-1)^2), "
                 ":80-102 (cosine 1 / 0), :144-159 (L2 sqrt(512), L1 512)",
        "dot_1_2": 1024.0,
        "l2sq_1_3": 2048.0,
        "l2_0_1": math.sqrt(512.0),
        "l1_0_1": 512.0,
        "cos_parallel": 1.0,
        "cos_orthogonal": 0.0,
        "tolerance": 0.001,
    },
    "batch_constant": {
        "_cite": "Vector512Tests.swift:174-204; MetalDistance512Tests.swift:50-66: "
                 "query 0 vs rows filled with i -> sqrt(512 i^2)",
        "first_two": [0.0, math.sqrt(512.0)],
        "tolerance": 0.001,
    },
    "distance_matrix": {
        "_cite": "MetalDistanceMatrixTests.swift:27-55 (symmetry, zero diagonal), "
                 ":76-111 (L2 sqrt(512), L1 512, cosine distance 0 for parallel)",
        "l2_0_1": math.sqrt(512.0),
        "l1_0_1": 512.0,
        "cos_parallel_distance": 0.0,
        "tolerance": 0.001,
    },
    "ivf_basic": {
        "_cite": "IVFIndexTests.swift:160-201: train on 8 4-d points, 4 centroids, "
                 "2 probes, insert (1,0,0,0) as vec1, query (0.9,0.1,0,0) -> vec1",
        "training": [[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0], [0, 0, 0, 1],
                     [0.5, 0.5, 0, 0], [0, 0.5, 0.5, 0], [0, 0, 0.5, 0.5], [0.5, 0, 0, 0.5]],
        "inserted": [1, 0, 0, 0],
        "query": [0.9, 0.1, 0, 0],
        "nprobe": 2,
        "expected_top1": "vec1",
    },
    "ivf_exact_self": {
        "_cite": "IVFIndexTests.swift:203-260: 32 clusters x 20 points, 128-d, insert "
                 "the first 100, .exact search for row 50 -> top-1 is vec50",
        "clusters": 32, "per_cluster": 20, "dim": 128, "inserted": 100,
        "query_row": 50, "k": 10,
    },
    "matrix_multiply": {
        "_cite": "MetalComponentTests.swift:244-271 and MetalComputeIntegrationTests.swift:"
                 "105-121: [[1,2,3],[4,5,6]] x [[7,8],[9,10],[11,12]] = [[58,64],[139,154]]",
        "a": [[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]],
        "b": [[7.0, 8.0], [9.0, 10.0], [11.0, 12.0]],
        "c": [[58.0, 64.0], [139.0, 154.0]],
        "tolerance": 0.001,
    },
    "sq8_roundtrip": {
        "_cite": "ScalarQuantizerTests.swift:55-74: int8 round trip of "
                 "[-1,-0.5,0,0.5,1] within 0.1",
        "vector": [-1.0, -0.5, 0.0, 0.5, 1.0],
        "tolerance": 0.1,
    },
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kats.json")
    with open(out, "w") as f:
        json.dump(KATS, f, indent=1)
    print("wrote", out)
