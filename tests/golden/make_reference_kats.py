"""Writes reference_kats.json: the known-answer vectors the reference's own
C++ shim tests assert (src/backend/mlx_metal/api_test.cc), transcribed as
data (inputs, dimension numbers, expected outputs) with their source lines.
Run: python tests/golden/make_reference_kats.py"""
import json
import pathlib

KATS = {
    # api_test.cc:624-687 — 2x2 dot, f16 and bf16 inputs {1,2,3,4}·{5,6,7,8}
    "dot_2x2": {"lhs": [[1, 2], [3, 4]], "rhs": [[5, 6], [7, 8]], "expected": [[19, 22], [43, 50]],
                "source": "api_test.cc:624-687"},
    # api_test.cc:930-1014 — f16 [2,2] {1,2,3,4} reduced over axis 1
    "reduce_f16": {"input": [[1, 2], [3, 4]], "sum": [3, 7], "max": [2, 4], "min": [1, 3],
                   "source": "api_test.cc:930-1014"},
    # api_test.cc:1016-1055 — two-output max/index over axis 1
    "argmax": {"input": [[1, 7, 7, 3], [-2, 5, 4, 5]], "values": [7, 5], "indices": [1, 1],
               "source": "api_test.cc:1016-1055"},
    # api_test.cc:1862-1905 — axis-0 gather of rows {2, 0} from [3,2] {1..6}
    "gather_axis0": {"operand": [[1, 2], [3, 4], [5, 6]], "indices": [2, 0], "expected": [[5, 6], [1, 2]],
                     "source": "api_test.cc:1862-1905"},
    # api_test.cc:1908-1945 — axis-1 gather of columns {1, 0}
    "gather_axis1": {"operand": [[1, 2], [3, 4], [5, 6]], "indices": [1, 0], "expected": [[2, 1], [4, 3], [6, 5]],
                     "source": "api_test.cc:1908-1945"},
    # api_test.cc:1949-1978 — point gather with start_index_map {0,1}
    "gather_point": {"operand": [[1, 2], [3, 4], [5, 6]], "indices": [[2, 1], [0, 0]], "expected": [6, 1],
                     "source": "api_test.cc:1949-1978"},
    # api_test.cc:2036-2090 — 1-D scatter set / add
    "scatter_1d": {"operand": [0, 10, 20, 30], "indices": [1, 3], "updates": [5, 7], "set": [0, 5, 20, 7],
                   "add": [0, 15, 20, 37], "source": "api_test.cc:2036-2090"},
    # api_test.cc:2092-2150 — point scatter into [3,2]
    "scatter_point": {"operand": [[1, 2], [3, 4], [5, 6]], "indices": [[2, 1], [0, 0]], "updates": [50, 60],
                      "set": [[60, 2], [3, 4], [5, 50]], "add": [[61, 2], [3, 4], [5, 56]],
                      "source": "api_test.cc:2092-2150"},
    # api_test.cc:2154-2222 — row-window scatter into [3,4]
    "scatter_window": {"operand": [[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]], "indices": [2, 0],
                       "updates": [[50, 60], [70, 80]],
                       "set": [[70, 80, 3, 4], [5, 6, 7, 8], [50, 60, 11, 12]],
                       "add": [[71, 82, 3, 4], [5, 6, 7, 8], [59, 70, 11, 12]],
                       "source": "api_test.cc:2154-2222"},
    # api_test.cc:2226-2308 — batched scatter set (operand/indices batching dim 0)
    "scatter_batched": {"operand_shape": [2, 3, 4], "operand": list(range(24)), "indices": [[[2], [0]], [[1], [2]]],
                        "updates": list(range(100, 116)),
                        "set": [104, 105, 106, 107, 4, 5, 6, 7, 100, 101, 102, 103, 12, 13, 14, 15,
                                108, 109, 110, 111, 112, 113, 114, 115],
                        "source": "api_test.cc:2226-2308"},
    # api_test.cc:271-309 — scaled-dot-product-attention custom call, f32,
    # q [1,1,2] ([q,h,hd]), k/v [2,1,2], token_index 0 (u32)
    "sdpa_one_head": {"q_shape": [1, 1, 2], "kv_shape": [2, 1, 2], "q": [1, 0], "k": [1, 0, 0, 1], "v": [10, 0, 0, 20],
                      "token_index": 0, "expected": [10, 0], "source": "api_test.cc:271-309"},
    # api_test.cc:311-352 — four query heads over two key/value heads
    "sdpa_grouped_heads": {"q_shape": [1, 4, 2], "kv_shape": [2, 2, 2], "q": [1, 0, 1, 0, 1, 0, 1, 0],
                           "k": [1, 0, 0, 1, 1, 0, 0, 1], "v": [10, 0, 20, 0, 0, 30, 0, 40], "token_index": 0,
                           "expected": [10, 0, 10, 0, 20, 0, 20, 0], "source": "api_test.cc:311-352"},
    # api_test.cc:2310-2360 — f32 [2,3] sorted along axis 1, its argsort, and
    # an s32 payload taken along that order
    "sort_kv": {"input": [[3, 1, 2], [6, 4, 5]], "sorted": [[1, 2, 3], [4, 5, 6]], "order": [[1, 2, 0], [1, 2, 0]],
                "values": [[10, 11, 12], [20, 21, 22]], "values_sorted": [[11, 12, 10], [21, 22, 20]],
                "source": "api_test.cc:2310-2360"},
}

if __name__ == "__main__":
    out = pathlib.Path(__file__).with_name("reference_kats.json")
    out.write_text(json.dumps(KATS, indent=1) + "\n")
    print(f"wrote {out}")
