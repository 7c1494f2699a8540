"""tokens_oracle.py -- pure-Python restatement of gguf-rs-cli's token-to-text
step and stop-token set.  TEST INFRASTRUCTURE ONLY: the checker for
include/gs_tokens.h; never called by the product.

Follows:
  build_byte_encoder      src/tokenizer/bpe.rs:199-208
  token_to_id             src/tokenizer/bpe.rs:37-38 (HashMap collect: the last
                          of equal strings wins)
  Tokenizer::decode       src/tokenizer/bpe.rs:180-197
  ChatTemplate::detect    src/tokenizer/chat.rs:9-24
  ChatTemplate::stop_tokens src/tokenizer/chat.rs:57-72
String::from_utf8_lossy is restated with Python's UTF-8 codec and
errors="replace", which substitutes U+FFFD for each maximal subpart of an
ill-formed sequence, the practice Rust documents; tests/test_tokens.py pins
that on the Unicode standard's own example.
"""

LLAMA, GPT2 = 0, 1
CHATML, LLAMA3, LLAMA2, GEMMA, PHI3, SIMPLE = range(6)


def byte_encoder():
    """bpe.rs:199-208: list of 256 chars, enc[b]."""
    enc = [None] * 256
    mapped = [False] * 256
    for lo, hi in ((33, 126), (161, 172), (174, 255)):
        for b in range(lo, hi + 1):
            enc[b] = chr(b)
            mapped[b] = True
    n = 0
    for b in range(256):
        if not mapped[b]:
            enc[b] = chr(256 + n)
            n += 1
    return enc


def token_to_id(vocab):
    d = {}
    for i, s in enumerate(vocab):
        d[s] = i
    return d


def decode(vocab, types, model, tid):
    """bpe.rs:180-197 -> str."""
    if tid >= len(vocab):
        return ""
    typ = types[tid] if tid < len(types) else 0
    if typ in (2, 3):
        return ""
    s = vocab[tid]
    if model == LLAMA:
        return s.replace("▁", " ")
    dec = {c: b for b, c in enumerate(byte_encoder())}
    bs = bytes(dec[c] for c in s if c in dec)
    if len(bs) == len(s):
        return bs.decode("utf-8", errors="replace")
    return s


def detect(vocab, tmpl):
    """chat.rs:9-24."""
    if tmpl is not None:
        for mark, kind in (("<|im_start|>", CHATML), ("<|start_header_id|>", LLAMA3),
                           ("<start_of_turn>", GEMMA), ("<|user|>", PHI3), ("[INST]", LLAMA2)):
            if mark in tmpl:
                return kind
    ids = token_to_id(vocab)
    for tok, kind in (("<|im_start|>", CHATML), ("<|eot_id|>", LLAMA3), ("<start_of_turn>", GEMMA),
                      ("<|user|>", PHI3), ("[INST]", LLAMA2)):
        if tok in ids:
            return kind
    return SIMPLE


def stop_tokens(vocab, kind, eos_ids):
    """chat.rs:57-72."""
    stops = list(eos_ids)
    extras = {CHATML: ["<|im_end|>", "<|endoftext|>"], LLAMA3: ["<|eot_id|>", "<|end_of_text|>"],
              GEMMA: ["<end_of_turn>"], PHI3: ["<|end|>"]}.get(kind, [])
    ids = token_to_id(vocab)
    for t in extras:
        if t in ids:
            stops.append(ids[t])
    return sorted(set(stops))
