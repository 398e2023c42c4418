"""Host side of `generate`: the reference's flag parsing (src/main.rs:65-155,
seed default at engine.rs:271) and the streaming decode of sampled ids
(tokenizer.rs:21-48, 260-360), without a GPU.

The streaming decoder is pinned by the reference's own unit tests
(tokenizer.rs:374-413), by the byte alphabet's asserted values, by the
tiny-gpt2 fixture vocabulary (tests/golden/tiny_gpt2/vocab.json, a data file
the reference's tests hold) and by the round trip of the reference's
tokenizer test texts (tests/engine.rs:58-72) split at every byte."""
import json
import os
import random

import numpy as np
import pytest

from conftest import ROOT

VOCAB = os.path.join(ROOT, "tests", "golden", "tiny_gpt2", "vocab.json")


# ---------------------------------------------------------------------------
# flags

def test_flag_reader_follows_main_rs():
    from nimbus_sampler.flags import Flags
    f = Flags.parse(["pos0", "--temperature", "-0.5", "--stream", "--top-p", "0.9", "tail",
                     "--json"])
    assert f.get("temperature") == "-0.5"      # a value may start with a single '-'
    assert f.has("stream") and f.get("stream") == ""
    assert f.get("top-p") == "0.9"
    assert f.positional == ["pos0", "tail"]
    assert f.has("json") and f.get("missing") is None
    g = Flags.parse(["--a", "--b", "x"])
    assert g.get("a") == "" and g.get("b") == "x"  # "--b" is not a value of --a


def test_generate_defaults_and_seed_rules():
    from nimbus_sampler.flags import DEFAULT_SEED, generate_params
    p, seed, _ = generate_params([])
    assert (p.max_new_tokens, p.temperature, p.top_k, p.top_p, p.repetition_penalty) == \
        (64, 0.0, 0, 1.0, 1.0)
    assert p.greedy() and p.seed is None and seed == DEFAULT_SEED == 0x5DEECE66D
    p, seed, _ = generate_params(["--seed", "7", "--temperature", "0.8", "--top-p", "0.9",
                                  "--top-k", "40", "--repetition-penalty", "1.3",
                                  "--max-new-tokens", "5"])
    assert seed == 7 and p.seed == 7 and p.top_k == 40 and p.max_new_tokens == 5
    assert p.temperature == float(np.float32(0.8)) == 0.800000011920929
    assert p.top_p == 0.8999999761581421 and p.repetition_penalty == float(np.float32(1.3))
    # `.and_then(|s| s.parse().ok())`: an unparsable seed is unset, not an error
    for bad in (["--seed"], ["--seed", "-1"], ["--seed", "7.5"], ["--seed", str(1 << 64)]):
        assert generate_params(bad)[1] == DEFAULT_SEED
    assert generate_params(["--seed", "+18446744073709551615"])[1] == (1 << 64) - 1
    from nimbus_sampler.flags import FlagError
    for bad in (["--temperature", "x"], ["--top-k", "-1"], ["--top-k", "1.0"], ["--max-new-tokens"]):
        with pytest.raises(FlagError):
            generate_params(bad)


def test_f32_parse_is_correctly_rounded():
    from nimbus_sampler.flags import FlagError, parse_f32
    # the f32 values of the configs' temperature and top-p fields
    for text, val in [("0.7", 0.699999988079071), ("0.8", 0.800000011920929),
                      ("0.9", 0.8999999761581421), ("0.95", 0.949999988079071),
                      ("0.99", 0.9900000095367432), ("1.3", 1.2999999523162842)]:
        assert float(parse_f32(text)) == val
    # just above the midpoint between 1 and 1 + 2^-23: the nearest f64 is the
    # midpoint itself, so rounding through f64 would give 1.0 (ties to even)
    assert float(parse_f32("1.00000005960464477539062500000001")) == 1.0 + 2.0 ** -23
    assert float(parse_f32("1.000000059604644775390625")) == 1.0  # the exact midpoint: even
    assert np.isinf(parse_f32("1e39")) and np.isinf(parse_f32("-INF")) and np.isnan(parse_f32("NaN"))
    assert float(parse_f32("3.4028235677973366e38")) == float(np.finfo(np.float32).max)
    assert np.isinf(parse_f32("3.4028235677973367e38"))  # at the overflow midpoint: to even = inf
    assert float(parse_f32("1e-50")) == 0.0 and str(parse_f32("-0.0")) == "-0.0"
    assert float(parse_f32("1e-45")) == float(np.float32(1e-45))  # the smallest subnormal
    for ok in (".5", "5.", "+3", "1E+2", "infinity"):
        parse_f32(ok)
    for bad in ("", " 1", "1 ", "1e", "e5", ".", "0x10", "1_0", "--1", "in",
                "1.5\n", "inf\n", "\u0663", "1\u0663.5"):
        with pytest.raises(FlagError):
            parse_f32(bad)
    # usize: ASCII digits only, the whole text (str::parse rejects a trailing
    # newline and non-ASCII digits such as ARABIC-INDIC DIGIT THREE)
    from nimbus_sampler.flags import parse_uint
    assert parse_uint("+5") == 5 and parse_uint("0") == 0
    for bad in ("5\n", "\u0663", "1\u0663", "", "+", "-1", " 5"):
        with pytest.raises(FlagError):
            parse_uint(bad)
    # random decimals: the nearest f32, checked against exact rationals
    import fractions
    rnd = random.Random(5)
    for _ in range(2000):
        text = f"{rnd.randint(0, 10**9)}.{rnd.randint(0, 10**12):012d}e{rnd.randint(-40, 38)}"
        got = parse_f32(text)
        exact = fractions.Fraction(text)
        if np.isinf(got):
            continue
        d = abs(fractions.Fraction(float(got)) - exact)
        for nb in (np.nextafter(got, np.float32(0)), np.nextafter(got, np.float32(np.inf))):
            if np.isfinite(nb):
                assert d <= abs(fractions.Fraction(float(nb)) - exact), text


# ---------------------------------------------------------------------------
# streaming decode

def test_byte_alphabet_matches_gpt2():
    # tokenizer.rs:374-383 (byte_alphabet_matches_gpt2)
    from nimbus_sampler.stream import byte_alphabet
    b2c, c2b = byte_alphabet()
    assert b2c[ord("!")] == 33 and b2c[0] == 256 and b2c[32] == 288 and b2c[173] == 323
    assert c2b[256] == 0 and c2b[33] == ord("!")
    assert sorted(b2c) == sorted(c2b) and len(set(b2c)) == 256


def test_utf8_stream_reference_unit_tests():
    from nimbus_sampler.stream import Utf8Stream
    # tokenizer.rs:394-406 (utf8_stream_never_splits_a_char)
    s = Utf8Stream()
    b = "你".encode("utf-8")
    assert s.push_bytes(b[:1]) == "" and s.push_bytes(b[1:2]) == "" and s.push_bytes(b[2:]) == "你"
    # tokenizer.rs:408-412 (utf8_stream_replaces_invalid_bytes)
    assert Utf8Stream().push_bytes(bytes([0xFF, ord("a")])) == "�a"
    # an announced sequence that is not UTF-8: one replacement for its bytes
    assert Utf8Stream().push_bytes(bytes([0xE4, 0x41, 0x42, 0x43])) == "�C"
    # ... which differs from decode()'s lossy whole-string conversion
    assert bytes([0xE4, 0x41, 0x2A]).decode("utf-8", errors="replace") == "�A*"
    s = Utf8Stream()
    assert s.push_bytes(bytes([0xE4, 0x41])) == "" and s.push_bytes(b"*") == "�"
    # a truncated tail is held back, and flushed lossily
    s = Utf8Stream()
    assert s.push_bytes("a".encode() + "€".encode()[:2]) == "a" and s.flush() == "�"
    assert s.flush() == ""


@pytest.mark.parametrize("text", [
    "hello world", "  spaces\tand\nnewlines  ", "中文混排 with emoji 😀!",
    "it's the engine's 123 tokens, don't you know?", "\u0000\u0001 control chars \u007f",
])
def test_fixture_vocab_streams_reference_texts(text):
    # the reference's round-trip texts (tests/engine.rs:58-72) as single-byte
    # tokens of the fixture vocabulary, pushed one by one: the stream never
    # emits part of a character, and the text comes back whole
    from nimbus_sampler.stream import IncrementalDecoder, TokenBytes
    table = TokenBytes.from_file(VOCAB)
    byte_tok = {}
    for i in range(len(table)):
        tb = table.token_bytes(i)
        if len(tb) == 1:
            byte_tok.setdefault(tb[0], i)
    assert len(byte_tok) == 256
    dec = IncrementalDecoder(table)
    out = []
    for byte in text.encode("utf-8"):
        d = dec.push(byte_tok[byte])
        d.encode("utf-8")  # a complete string
        out.append(d)
    out.append(dec.flush())
    assert "".join(out) == text


def test_fixture_vocab_multi_byte_tokens():
    from nimbus_sampler.stream import IncrementalDecoder, TokenBytes
    with open(VOCAB, encoding="utf-8") as f:
        vocab = json.load(f)
    table = TokenBytes(vocab)
    assert table.token_bytes(vocab["Ġnimbus"]) == b" nimbus"
    assert table.token_bytes(vocab["nimbus"]) == b"nimbus"
    assert table.token_bytes(len(table) + 5) == b""  # unknown id: no bytes
    dec = IncrementalDecoder(table)
    assert dec.push(vocab["nimbus"]) + dec.push(vocab["Ġnimbus"]) + dec.flush() == "nimbus nimbus"


def test_batch_streams_skip_finished_sequences():
    from nimbus_sampler.stream import BatchStreams, TokenBytes
    table = TokenBytes.from_file(VOCAB)
    with open(VOCAB, encoding="utf-8") as f:
        vocab = json.load(f)
    bs = BatchStreams(table, 2)
    n = vocab["nimbus"]
    bs.push_step([n, n], [True, False])
    bs.push_step([n, n], [True, True])
    bs.flush()
    assert bs.text == ["nimbusnimbus", "nimbus"]
