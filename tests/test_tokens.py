"""Token id -> text and the stop-token set (include/gs_tokens.h): the host
text step after the sampler (src/tokenizer/bpe.rs:180-208,
src/tokenizer/chat.rs:9-72).  Host code only: these run on the CPU.

The oracle (oracle/tokens_oracle.py) is pinned by facts it does not compute
itself: the Unicode standard's example of U+FFFD substitution per maximal
subpart (what String::from_utf8_lossy documents), GPT-2's published
byte-to-character table, and hand-worked tokens.  The C ABI must then equal
the oracle on every id of randomised vocabularies.
"""
import numpy as np
import pytest

import tokens_oracle as T


# ---- oracle pins -------------------------------------------------------------
def test_lossy_utf8_is_maximal_subpart_substitution():
    """Unicode 15, section 3.9, Table 3-8: <61 F1 80 80 E1 80 C2 62 80 63 80 BF 64>
    decodes to 0061 FFFD FFFD FFFD 0062 FFFD 0063 FFFD FFFD 0064."""
    b = bytes([0x61, 0xF1, 0x80, 0x80, 0xE1, 0x80, 0xC2, 0x62, 0x80, 0x63, 0x80, 0xBF, 0x64])
    assert b.decode("utf-8", errors="replace") == "a���b�c��d"
    # surrogates and overlongs are ill-formed byte by byte
    assert b"\xed\xa0\x80".decode("utf-8", errors="replace") == "�" * 3
    assert b"\xc0\xaf".decode("utf-8", errors="replace") == "�" * 2
    assert b"\xf4\x90\x80\x80".decode("utf-8", errors="replace") == "�" * 4


def test_byte_encoder_table():
    """GPT-2's byte-level table: printable Latin-1 maps to itself, the other
    68 bytes to U+0100.. in byte order (space = U+0120 'Ġ', newline = U+010A 'Ċ')."""
    enc = T.byte_encoder()
    assert len(set(enc)) == 256
    assert enc[ord("a")] == "a" and enc[ord("~")] == "~" and enc[0xE4] == "ä"
    assert enc[0] == "Ā" and enc[10] == "Ċ" and enc[32] == "Ġ"
    assert enc[0x7F] == "ġ" and enc[0xAD] == "Ń"
    assert sorted(ord(c) for c in enc if ord(c) >= 256) == list(range(256, 324))


def test_decode_worked_examples():
    vocab = ["Ġhello", "ĊĊ", "ä¸", "ä¸Ń", "▁x", "<|im_end|>", "a▁b"]
    types = [1, 1, 1, 1, 1, 3, 1]
    g = lambda i: T.decode(vocab, types, T.GPT2, i)
    assert g(0) == " hello"
    assert g(1) == "\n\n"
    assert g(2) == "�"                    # E4 B8: a truncated 3-byte sequence
    assert g(3) == "中"                        # E4 B8 AD (0xAD is 'Ń' in the table)
    assert g(4) == "▁x"                   # U+2581 is not in the byte table: token unchanged
    assert g(5) == ""                          # control / special type
    assert g(99) == ""
    ll = lambda i: T.decode(vocab, types, T.LLAMA, i)
    assert ll(4) == " x" and ll(6) == "a b" and ll(0) == "Ġhello"


def test_stop_tokens_and_detect_examples():
    vocab = ["a", "<|im_start|>", "<|im_end|>", "<|endoftext|>", "<|im_end|>", "<end_of_turn>"]
    assert T.token_to_id(vocab)["<|im_end|>"] == 4              # the last duplicate
    assert T.detect(vocab, None) == T.CHATML
    assert T.detect(vocab, "{% [INST] %}") == T.LLAMA2
    assert T.detect(["x"], None) == T.SIMPLE
    assert T.stop_tokens(vocab, T.CHATML, [7, 3, 7]) == [3, 4, 7]
    assert T.stop_tokens(vocab, T.GEMMA, []) == [5]
    assert T.stop_tokens(vocab, T.LLAMA2, [2]) == [2]


# ---- C ABI against the oracle -------------------------------------------------
def _random_vocab(rng, n, model):
    enc = T.byte_encoder()
    vocab, types = [], []
    for i in range(n):
        r = rng.random()
        if model == T.GPT2 and r < 0.8:
            if rng.random() < 0.5:
                bs = bytes(rng.integers(0, 256, rng.integers(1, 7)).astype(np.uint8))
            else:                                                     # UTF-8 text, cut anywhere
                txt = "héllo 中文 \n ok".encode()
                a = int(rng.integers(0, len(txt)))
                bs = txt[a:a + int(rng.integers(1, 7))]
            vocab.append("".join(enc[b] for b in bs))
        elif r < 0.9:
            vocab.append("▁" + "".join(rng.choice(list("abcxyzé中▁"), rng.integers(0, 5))))
        else:
            vocab.append(rng.choice(["<|im_start|>", "<|im_end|>", "<|endoftext|>", "<|eot_id|>",
                                     "<start_of_turn>", "<end_of_turn>", "[INST]", "<|end|>", "<s>"]))
        types.append(int(rng.choice([1, 1, 1, 2, 3, 4, 6])))
    return vocab, types[: n - 7]                                       # a few types missing: read 0


@pytest.mark.parametrize("model", [0, 1])
def test_decode_matches_oracle(model):
    import gs_sampler
    rng = np.random.default_rng(11 + model)
    vocab, types = _random_vocab(rng, 3000, model)
    v = gs_sampler.Vocab(vocab, types, model)
    for i in range(len(vocab) + 3):
        want = T.decode(vocab, types, model, i).encode("utf-8", errors="surrogatepass")
        assert v.decode_bytes(i) == want, (i, vocab[i] if i < len(vocab) else None)
    ids = rng.integers(0, len(vocab) + 5, 500)
    want = "".join(T.decode(vocab, types, model, int(i)) for i in ids)
    assert v.decode(ids) == want
    for s in set(vocab[:200]) | {"<|im_end|>", "missing"}:
        assert v.find(s) == T.token_to_id(vocab).get(s)
    for tmpl in (None, "<|im_start|>", "x<|start_header_id|>y", "<start_of_turn>", "<|user|>", "[INST]", ""):
        assert v.detect(tmpl) == T.detect(vocab, tmpl)
    for kind in range(6):
        eos = [int(x) for x in rng.integers(0, 100, 3)]
        assert v.stop_tokens(kind, eos) == T.stop_tokens(vocab, kind, eos)
    v.close()


def test_vocab_arguments_rejected():
    import ctypes
    import gs_sampler
    lib = gs_sampler.load_library()
    h = ctypes.c_void_p()
    assert lib.gs_vocab_create(None, None, 0, None, 0, 2, ctypes.byref(h)) == gs_sampler.GS_ERR_INVALID
    off = np.array([0, 5, 3], np.uint64)                            # decreasing offsets
    assert lib.gs_vocab_create(b"abcde", off.ctypes.data, 2, None, 0, 0, ctypes.byref(h)) == gs_sampler.GS_ERR_INVALID
    v = gs_sampler.Vocab([], [], 0)
    assert v.decode_bytes([0, 1]) == b"" and v.detect() == gs_sampler.TMPL_SIMPLE
