"""Split-model index and tensor row ranges on the CPU: ModelIndex::new /
tensor / inventory (frontier_gguf.rs:101-137) and Tensor::rows / expert
(:86-98), with the cases of the reference's tests (frontier_gguf.rs:225-236,
265-288) restated on synthetic shards: the reference's header fixtures
(reference/q3-metadata.gguf, shard2/3-header.gguf) are not in its tree here."""
import numpy as np
import pytest

import uq
import gguf_writer as W

U64_MAX = (1 << 64) - 1


def gerr(fn, *args):
    with pytest.raises(uq.GgufError) as e:
        fn(*args)
    assert e.value.status == uq.Error.FORMAT
    return e.value.gguf_error


def shard(no, count, total, tensors, extra=()):
    meta = [("split.no", W.U16, no), ("split.count", W.U16, count), ("split.tensors.count", W.I32, total)]
    data, _ = W.write(meta + list(extra), tensors)
    return uq.Gguf.parse(data, len(data))


def q4k(dims):
    return bytes(W.tensor_bytes(12, dims))


def test_rows_and_expert_ranges():
    # a rank-3 expert tensor [256 values, 4 rows, 5 experts] of Q4_K (144 B rows)
    g = shard(0, 1, 2, [("blk.0.ffn_gate_exps.weight", [256, 4, 5], 12, q4k([256, 4, 5])),
                        ("blk.0.attn_q.weight", [256, 3], 12, q4k([256, 3]))])
    t = g.tensors()
    e = 0 if t[0]["dims"] == [256, 4, 5] else 1
    d = 1 - e
    off, nb = t[e]["offset"], t[e]["bytes"]
    total = nb // 144
    assert g.rows(e, 0, total) == (off, nb)
    assert gerr(g.rows, e, total, 1) == "TensorBounds"
    assert gerr(g.rows, e, 0, 0) == "TensorBounds"
    assert gerr(g.rows, e, U64_MAX, 2) == "Overflow"
    assert g.rows(e, 3, 2) == (off + 3 * 144, 2 * 144)
    first, last = g.expert(e, 0), g.expert(e, 4)
    assert first == (off, 4 * 144)
    assert last[0] + last[1] == off + nb
    assert g.expert(e, 2) == (off + 8 * 144, 4 * 144)
    assert gerr(g.expert, e, 5) == "Shape"
    assert gerr(g.expert, d, 0) == "Shape"           # rank 2: no experts


def model_shards():
    s0 = shard(0, 3, 4, [], extra=[("general.architecture", W.STRING, "qwen2moe")])
    s1 = shard(1, 3, 4, [("per_layer_token_embd.weight", [256, 2], 12, q4k([256, 2])),
                         ("blk.0.attn_q.weight", [256, 3], 12, q4k([256, 3]))])
    s2 = shard(2, 3, 4, [("blk.0.ffn_up_exps.weight", [256, 2, 4], 12, q4k([256, 2, 4])),
                         ("blk.0.ffn_down_exps.weight", [256, 2, 4], 12, q4k([256, 2, 4]))])
    return s0, s1, s2


def test_whole_model_directory():
    s0, s1, s2 = model_shards()
    ix = uq.GgufIndex([s2, s0, s1])                    # any order: ModelIndex::new sorts by split.no
    assert [s.split()[0] for s in ix.shards] == [0, 1, 2]
    assert ix.inventory() == [3 * 144, 2 * 144, 2 * 8 * 144]
    sh, ti = ix.find("per_layer_token_embd.weight")
    assert sh == 1 and ix.shards[sh].tensors()[ti]["name"] == "per_layer_token_embd.weight"
    sh, ti = ix.find("blk.0.ffn_down_exps.weight")
    assert sh == 2 and ix.shards[sh].expert(ti, 3)[1] == 2 * 144
    assert gerr(ix.find, "blk.9.attn_q.weight") == "Missing"
    # a missing shard, a duplicate name, a disagreeing count, a wrong total
    assert gerr(uq.GgufIndex, [s0, s1]) == "Split"
    assert gerr(uq.GgufIndex, []) == "Split"
    dup = shard(2, 3, 4, [("blk.0.attn_q.weight", [256, 3], 12, q4k([256, 3])),
                          ("blk.0.ffn_down_exps.weight", [256, 2, 4], 12, q4k([256, 2, 4]))])
    assert gerr(uq.GgufIndex, [s0, s1, dup]) == "Duplicate"
    other = shard(2, 4, 4, [("blk.0.ffn_up_exps.weight", [256, 2, 4], 12, q4k([256, 2, 4])),
                            ("blk.0.ffn_down_exps.weight", [256, 2, 4], 12, q4k([256, 2, 4]))])
    assert gerr(uq.GgufIndex, [s0, s1, other]) == "Split"
    short = shard(2, 3, 4, [("blk.0.ffn_up_exps.weight", [256, 2, 4], 12, q4k([256, 2, 4]))])
    assert gerr(uq.GgufIndex, [s0, s1, short]) == "Split"  # 3 names, split.tensors.count 4
    twice = shard(1, 3, 4, [])
    assert gerr(uq.GgufIndex, [s0, twice, s1]) == "Split"  # split.no 1 twice
