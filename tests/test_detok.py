"""Token ids -> text (qwen_hip_vocab_*) against the reference tokenizer's
decode compiled from its sources (oracle/_ref: qwen_tokenizer_load /
qwen_tokenizer_decode, qwen_asr_tokenizer.c:500-609) on the same vocab.json,
and the transcript rule of the reference's greedy loop (qwen_asr.c:729-754)
restated from the reference's constants."""
import ctypes as C
import json

import numpy as np
import pytest

ASR_TEXT, EOT, IM_END = 151704, 151643, 151645


def byte_level_table():
    """GPT-2 byte -> code point (the public bytes_to_unicode rule)."""
    keep = list(range(33, 127)) + list(range(161, 173)) + list(range(174, 256))
    cps, extra = {}, 0
    for b in range(256):
        if b in keep:
            cps[b] = b
        else:
            cps[b] = 256 + extra
            extra += 1
    return cps


def encode_key(bs, table):
    return "".join(chr(table[b]) for b in bs)


@pytest.fixture(scope="module")
def vocab_file(tmp_path_factory):
    table = byte_level_table()
    r = np.random.default_rng(7)
    entries = {}
    # every single byte, a space-prefixed word, multi-byte UTF-8 text
    for b in range(256):
        entries[encode_key(bytes([b]), table)] = b
    words = ["hello", " world", " café", "你好", " über", "\n", "\t\t", "a\u0000b"]
    for i, w in enumerate(words):
        entries[encode_key(w.encode("utf-8"), table)] = 300 + i
    for i in range(200):   # random byte strings
        entries[encode_key(bytes(r.integers(0, 256, r.integers(1, 7)).tolist()), table)] = 400 + i
    # keys the table does not cover: plain ASCII space (cp 32), a 4-byte code point, a code point > 511
    entries[" x"] = 700
    entries["\U0001F600"] = 701
    entries["؀z"] = 702
    path = tmp_path_factory.mktemp("vocab") / "vocab.json"
    # one file with \\u escapes (json.dumps default) and one with raw UTF-8
    path.write_text(json.dumps(entries, ensure_ascii=True))
    raw = path.parent / "vocab_raw.json"
    raw.write_text(json.dumps(entries, ensure_ascii=False), encoding="utf-8")
    return path, raw, entries


def ref_tokenizer(P):
    ref = P.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    if not hasattr(ref, "qwen_tokenizer_load"):
        pytest.skip("oracle/_ref built without the tokenizer")
    ref.qwen_tokenizer_load.restype = C.c_void_p
    ref.qwen_tokenizer_load.argtypes = [C.c_char_p]
    ref.qwen_tokenizer_decode.restype = C.c_char_p
    ref.qwen_tokenizer_decode.argtypes = [C.c_void_p, C.c_int]
    ref.qwen_tokenizer_free.argtypes = [C.c_void_p]
    return ref


@pytest.mark.parametrize("which", [0, 1])
def test_pieces_match_reference(P, qa, vocab_file, which):
    path = vocab_file[which]
    ref = ref_tokenizer(P)
    rt = ref.qwen_tokenizer_load(str(path).encode())
    assert rt
    v = qa.Vocab(str(path))
    try:
        assert len(v) == 703
        for i in range(-2, 760):
            assert v.piece(i) == ref.qwen_tokenizer_decode(rt, i), i
    finally:
        ref.qwen_tokenizer_free(rt)
        v.close()


def test_pieces_are_the_bytes(qa, vocab_file):
    path, _, _ = vocab_file
    v = qa.Vocab(str(path))
    assert v.piece(ord("A")) == b"A" and v.piece(32) == b" " and v.piece(305) == b"\n"
    assert v.piece(10) == b""              # the "\n" word re-keyed byte 10's entry to id 305
    assert v.piece(301) == " world".encode() and v.piece(302) == " café".encode()
    assert v.piece(303) == "你好".encode()
    assert v.piece(307) == b"a"            # C string: the piece ends at its NUL byte, as the reference's
    assert v.piece(700) == b"?x"           # ' ' (U+0020) is not in the byte-level table
    assert v.piece(701) == b"??"           # written as a \ud83d\ude00 surrogate pair: two code points
    assert v.piece(702) == b"?z"
    assert v.piece(EOT) == b"" and v.piece(10**6) == b""


def test_transcript_rule(qa, vocab_file):
    path, _, _ = vocab_file
    v = qa.Vocab(str(path))
    hello, world = 300, 301
    # before <asr_text> nothing is emitted (language tag etc.); EOS ends the text
    assert v.transcript([ord("e"), ord("n"), ASR_TEXT, hello, world, IM_END, hello]) == b"hello world"
    assert v.transcript([hello, world]) == b""
    assert v.transcript([hello, world], past_asr_text=True) == b"hello world"
    assert v.transcript([ASR_TEXT, hello, EOT, world]) == b"hello"
    assert v.transcript([]) == b""


def test_vocab_errors(qa, tmp_path):
    with pytest.raises(RuntimeError, match="cannot open"):
        qa.Vocab(str(tmp_path / "missing.json"))
    bad = tmp_path / "v.json"
    bad.write_text('["not", "an", "object"]')
    with pytest.raises(RuntimeError, match="not a JSON object"):
        qa.Vocab(str(bad))
    bad.write_text('{"a": 1, "b": }')
    with pytest.raises(RuntimeError, match="not a JSON object"):
        qa.Vocab(str(bad))
