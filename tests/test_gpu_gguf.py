"""A Qwen2 model loaded from a GGUF file (uq_gguf_open + uq_model_load_gguf)
decodes exactly like the same tensors set one by one (uq_model_set_tensor):
same logits bits, same greedy ids. A file without output.weight (tied
embeddings) uses token_embd.weight as the output matrix."""
import numpy as np
import pytest

import uq
import gguf_writer as W

CFG = dict(layers=2, dim=256, hidden=512, heads=4, kv_heads=2, head_dim=64, vocab=1024, max_seq=128,
           eps=1e-6, theta=1e6)


@pytest.fixture(scope="module")
def gpu():
    uq.init(0)
    yield


def run(m, steps=12):
    first = m.decode_step(7, 0)
    logits = m.logits()
    ids, _ = m.decode_run(first, 1, steps)
    return first, logits, ids


@pytest.mark.gpu
@pytest.mark.parametrize("tie", [False, True])
def test_gguf_model_matches_direct_tensors(gpu, tmp_path, tie):
    tensors = uq.synth_qwen2(CFG, 0x5EED00AA)
    if tie:
        tensors["output.weight"] = tensors["token_embd.weight"]
    data, _ = W.qwen2_file(CFG, tensors, tie_output=tie)
    p = tmp_path / "qwen2.gguf"
    p.write_bytes(data)
    ref = uq.Qwen2Model(CFG, tensors)
    got = uq.Qwen2Model.from_gguf(str(p), CFG["max_seq"])
    f0, l0, i0 = run(ref)
    f1, l1, i1 = run(got)
    assert f0 == f1
    assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32))
    assert np.array_equal(i0, i1)
    ref.free()
    got.free()


@pytest.mark.gpu
def test_gguf_model_rejects_unsupported_kinds(gpu, tmp_path):
    tensors = uq.synth_qwen2(CFG, 0x5EED00AB)
    kind, n, rows, arr = tensors["blk.0.ffn_up.weight"]
    # same bytes declared as Q4_K rows (144 B per 256 values): the dense decoder takes Q8_0 only
    raw = arr.tobytes()
    q4_rows = len(raw) // (n // 256 * 144)
    meta_cfg = dict(CFG)
    data, _ = W.write([("general.architecture", W.STRING, "qwen2")],
                      [("blk.0.ffn_up.weight", [n, q4_rows], 12, raw[:q4_rows * (n // 256 * 144)])])
    p = tmp_path / "bad.gguf"
    p.write_bytes(data)
    g = uq.Gguf.open(str(p))
    m = uq.Qwen2Model(meta_cfg)
    with pytest.raises(uq.UqError) as e:
        uq._check(uq.lib().uq_model_load_gguf(m.handle, g.handle))
    assert e.value.status == uq.Error.QUANT_TYPE
    m.free()
    g.free()
