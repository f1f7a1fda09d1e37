"""Writes routing_cases.json: edge cases of top-k selection and of the stable
expert sort, with expected answers computed by brute force in plain Python
(no torch, no oracle). Cases follow the reference tests' edge cases: all-tied
logits (test_router_all_groups.py tied=True), ties at the top, an empty
expert and a single heavy expert (test_block_fp8_transpose_gemm.py COUNTS).

Run: python tests/golden/make_routing_cases.py
"""

import json
import math
import os


def brute_topk(values, k):
    return sorted(range(len(values)), key=lambda e: (-values[e], e))[:k]


def softmax(v):
    m = max(v)
    ex = [math.exp(x - m) for x in v]
    s = sum(ex)
    return [x / s for x in ex]


def route_case(name, logits, top_k, mode):
    ids = []
    for row in logits:
        values = softmax(row) if mode == "softmax_then_topk" else row
        ids.append(brute_topk(values, top_k))
    return dict(name=name, logits=logits, top_k=top_k, mode=mode, ids=ids)


def sort_case(name, ids, experts):
    flat = [e for row in ids for e in row]
    order = sorted(range(len(flat)), key=lambda i: (flat[i], i))
    counts = [flat.count(e) for e in range(experts)]
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    slots = [0] * len(flat)
    for pos, i in enumerate(order):
        slots[i] = pos
    return dict(name=name, ids=ids, experts=experts, order=order, offsets=offsets, slots=slots)


def main():
    route = [
        route_case("all tied", [[0.0] * 8, [1.5] * 8], 3, "topk_then_softmax"),
        route_case("tie at top", [[0.1, 2.0, -1.0, 2.0, 0.5, 2.0]], 2, "topk_then_softmax"),
        route_case("tie softmax", [[3.0, -1.0, 3.0, 0.0]], 2, "softmax_then_topk"),
        route_case("negative", [[-5.0, -1.0, -3.0, -1.0, -2.0]], 4, "topk_then_softmax"),
        route_case("k equals E", [[0.3, -0.2, 0.9]], 3, "topk_then_softmax"),
    ]
    sort = [
        sort_case("empty expert", [[0, 2], [2, 0], [3, 2]], 5),
        sort_case("one heavy expert", [[1, 0], [1, 2], [1, 3], [1, 0]], 4),
        sort_case("single token", [[3, 1, 2]], 4),
    ]
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "routing_cases.json")
    with open(path, "w") as f:
        json.dump(dict(route=route, sort=sort), f, indent=1)


if __name__ == "__main__":
    main()
