"""Streaming decode of sampled ids on the host (the step after the sampler
in `generate --stream`).

The reference turns each sampled id into bytes through the GPT-2 byte-level
alphabet (tokenizer.rs:21-48, token_bytes at tokenizer.rs:260-268) and feeds
them to a UTF-8 stream that only ever emits whole characters
(IncrementalDecoder / Utf8Stream, tokenizer.rs:279-360), driven once per
generated token by Engine::generate_stream (engine.rs:296-316).

`BatchStreams` does the same for B sequences at once: after each device
decode step the host reads the step's B tokens (4 B each) and the done flags,
and every live sequence's decoder receives its token.
"""
import json
from typing import Dict, List, Optional, Sequence

REPLACEMENT = "�"


def byte_alphabet():
    """GPT-2's reversible byte <-> printable code point map (tokenizer.rs:27-48):
    the 188 printable bytes keep their value, the others take 256, 257, ...
    in byte order.  Returns (byte_to_code[256], code_to_byte dict)."""
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    base = len(bs)
    for b in range(256):
        if b not in bs:
            bs.append(b)
    byte_to_code = [0] * 256
    code_to_byte: Dict[int, int] = {}
    for off, b in enumerate(bs):
        code = b if off < base else 256 + (off - base)
        byte_to_code[b] = code
        code_to_byte[code] = b
    return byte_to_code, code_to_byte


class TokenBytes:
    """id -> raw bytes of a byte-level BPE vocabulary (tokenizer.rs:260-268):
    each character of the token string maps back through the alphabet, a
    character outside it is dropped, an unknown id has no bytes."""

    def __init__(self, vocab: Dict[str, int]):
        _, code_to_byte = byte_alphabet()
        n = max(vocab.values()) + 1 if vocab else 0
        table: List[bytes] = [b""] * n
        for tok, i in vocab.items():
            table[i] = bytes(code_to_byte[ord(c)] for c in tok if ord(c) in code_to_byte)
        self.table = table

    @classmethod
    def from_file(cls, path: str) -> "TokenBytes":
        with open(path, "rb") as f:
            return cls(json.loads(f.read().decode("utf-8")))

    def __len__(self) -> int:
        return len(self.table)

    def token_bytes(self, token_id: int) -> bytes:
        return self.table[token_id] if 0 <= token_id < len(self.table) else b""


def _utf8_len(first: int) -> int:
    """Length of the sequence a lead byte announces; 0: continuation / invalid
    (tokenizer.rs:352-360)."""
    if first <= 0x7F:
        return 1
    if 0xC0 <= first <= 0xDF:
        return 2
    if 0xE0 <= first <= 0xEF:
        return 3
    if 0xF0 <= first <= 0xF7:
        return 4
    return 0


class Utf8Stream:
    """Utf8Stream (tokenizer.rs:302-350): buffers a truncated trailing
    sequence until the bytes that complete it arrive; an invalid lead byte,
    or an announced sequence that is not valid UTF-8, becomes one U+FFFD."""

    def __init__(self):
        self.buffer = bytearray()

    def push_bytes(self, data: bytes) -> str:
        self.buffer += data
        return self._take_complete()

    def flush(self) -> str:
        out = bytes(self.buffer).decode("utf-8", errors="replace") if self.buffer else ""
        self.buffer.clear()
        return out

    def _take_complete(self) -> str:
        out: List[str] = []
        while self.buffer:
            need = _utf8_len(self.buffer[0])
            if need == 0:
                out.append(REPLACEMENT)
                del self.buffer[0]
                continue
            if len(self.buffer) < need:
                break  # wait for the rest of the sequence
            try:
                out.append(bytes(self.buffer[:need]).decode("utf-8"))
            except UnicodeDecodeError:
                out.append(REPLACEMENT)
            del self.buffer[:need]
        return "".join(out)


class IncrementalDecoder:
    """IncrementalDecoder (tokenizer.rs:286-300): push a token id, receive
    only the characters it completes; flush at the end."""

    def __init__(self, table: TokenBytes):
        self.table = table
        self.stream = Utf8Stream()

    def push(self, token_id: int) -> str:
        return self.stream.push_bytes(self.table.token_bytes(token_id))

    def flush(self) -> str:
        return self.stream.flush()


class BatchStreams:
    """One IncrementalDecoder per sequence of a device-resident decode loop."""

    def __init__(self, table: TokenBytes, batch: int):
        self.decoders = [IncrementalDecoder(table) for _ in range(batch)]
        self.text = [""] * batch

    def push_step(self, tokens: Sequence[int], live: Optional[Sequence[bool]] = None) -> List[str]:
        """Feed one step's tokens (sequence b only if live[b]); returns each
        sequence's new text."""
        deltas = []
        for b, dec in enumerate(self.decoders):
            d = dec.push(int(tokens[b]) & 0xFFFFFFFF) if (live is None or live[b]) else ""
            self.text[b] += d
            deltas.append(d)
        return deltas

    def flush(self) -> List[str]:
        out = []
        for b, dec in enumerate(self.decoders):
            d = dec.flush()
            self.text[b] += d
            out.append(d)
        return out
