"""Detokenization (Model::text, driver/src/llm.rs:87-99) and the prompt files of
the reference's generate harness (llm.rs:396-447), on the CPU.

The byte map is pinned by GPT-2's published byte-level convention, which
Model::text inverts: printable bytes 33-126, 161-172 and 174-255 are their own
characters, the other 68 bytes are U+0100.. in ascending order (so space is
"Ġ" U+0120, newline "Ċ" U+010A, tab "ĉ" U+0109), and every one of the 256
bytes round-trips."""
import os

import numpy as np
import pytest

import gguf_writer as W
import uq
import evalrun

HERE = os.path.dirname(os.path.abspath(__file__))
PROMPTS = os.path.join(HERE, "golden", "prompts")


def gpt2_byte_char(b):
    """GPT-2 bytes_to_unicode, written from its published definition."""
    printable = list(range(33, 127)) + list(range(161, 173)) + list(range(174, 256))
    if b in printable:
        return chr(b)
    others = [x for x in range(256) if x not in printable]
    return chr(256 + others.index(b))


def vocab_file(tokens):
    data, _ = W.write([("tokenizer.ggml.tokens", W.ARRAY, (W.STRING, tokens))], [])
    return uq.Gguf.parse(np.frombuffer(data, np.uint8), len(data))


def test_known_gpt2_characters():
    g = vocab_file(["Ġhello", "Ċ", "ĉ", "ĠThe", "Ā", "Ń", "ń", "abc"])
    assert g.token_bytes(0) == b" hello"
    assert g.token_bytes(1) == b"\n"
    assert g.token_bytes(2) == b"\t"
    assert g.token_bytes(3) == b" The"
    assert g.token_bytes(4) == b"\x00"                 # U+0100: the first unprintable byte
    assert g.token_bytes(5) == b"\xad"                 # U+0143: the 68th, soft hyphen 173
    assert g.token_bytes(6) == "ń".encode()           # U+0144: past the map, its own UTF-8
    assert g.token_bytes(7) == b"abc"
    assert g.text(0) == " hello"


def test_all_bytes_round_trip():
    chars = [gpt2_byte_char(b) for b in range(256)]
    assert len(set(chars)) == 256
    g = vocab_file(chars + ["".join(chars[b] for b in b"caf\xc3\xa9")])
    for b in range(256):
        assert g.token_bytes(b) == bytes([b]), b
    assert g.text(256) == "café"                      # multi-byte UTF-8 rebuilt from byte characters


def test_lossy_text_of_a_partial_character():
    # one byte of a two-byte UTF-8 sequence: the reference's from_utf8_lossy gives U+FFFD
    g = vocab_file([gpt2_byte_char(0xC3)])
    assert g.token_bytes(0) == b"\xc3"
    assert g.text(0) == "�"


def test_token_text_errors():
    g = vocab_file(["a"])
    with pytest.raises(uq.UqError):
        g.token_bytes(1)                                # index out of range
    data, _ = W.write([("general.architecture", W.STRING, "qwen2")], [])
    with pytest.raises(uq.UqError):
        uq.Gguf.parse(np.frombuffer(data, np.uint8), len(data)).token_bytes(0)   # no tokenizer


def test_reference_prompt_files():
    lens = {}
    for label in evalrun.LABELS:
        ids = evalrun.read_tokens(os.path.join(PROMPTS, "prompt_%s.tokens" % label))
        lens[label] = len(ids)
        assert ids[0] == 151644                         # <|im_start|>
        assert (ids < 151936).all()
        assert len(ids) + evalrun.max_new_for(label) < 1024
    assert lens == {"sentence": 28, "riddle": 53, "scale": 139}
    assert evalrun.max_new_for("scale") == 512 and evalrun.max_new_for("riddle") == 160


def test_read_tokens_rejects_bad_count(tmp_path):
    p = tmp_path / "bad.tokens"
    p.write_bytes(np.array([3, 1, 2], np.uint32).tobytes())
    with pytest.raises(ValueError):
        evalrun.read_tokens(str(p))
