"""GPU test of `generate`: the reference's generate flags (main.rs:147-155)
drive the device decode loop (nis_lm_head_logits -> nis_decode_step), and the
ids stream through the byte-level decoder (tokenizer.rs:279-360).

Checks: every sequence's ids equal the oracle's sample() loop over the same
device logits, with the history as the penalty list and Rng(seed + b)
(boundary rows end the comparison of their sequence, as in the decode test);
the streamed text equals one push of all the ids' bytes (and decode() when
those bytes are valid UTF-8)."""
import io
import os

import numpy as np
import pytest

from conftest import ROOT
from parity_util import BOUNDARY

pytestmark = pytest.mark.gpu

VOCAB = os.path.join(ROOT, "tests", "golden", "tiny_gpt2", "vocab.json")


@pytest.mark.parametrize("argv", [
    ["--max-new-tokens", "6", "--temperature", "0.8", "--top-p", "0.9", "--seed", "11"],
    ["--max-new-tokens", "5", "--temperature", "0.7", "--top-k", "40",
     "--repetition-penalty", "1.3"],                              # default seed
    ["--max-new-tokens", "6", "--repetition-penalty", "1.2"],     # greedy with a penalty
    ["--max-new-tokens", "4", "--temperature", "1", "--seed", "not-a-number"],
])
def test_generate_matches_oracle_loop(argv):
    from nimbus_sampler import cli
    from nimbus_sampler.stream import TokenBytes, Utf8Stream
    from oracle import oracle
    out = io.StringIO()
    args = argv + ["--vocab", VOCAB, "--batch", "8", "--hidden", "64", "--stream"]
    print(f"[generate] {' '.join(args)}", flush=True)
    res = cli.generate(args, out=out, keep_logits=True)
    params, seed, ids = res["params"], res["seed"], res["ids"]
    n = params.max_new_tokens
    assert len(res["logits"]) == n and all(len(x) == n for x in ids)
    p = oracle.make_params(params.temperature, params.top_p, params.top_k,
                           params.repetition_penalty)
    diverged = 0
    for b in range(8):
        rng = oracle.Rng(seed + b)
        hist = []
        for s in range(n):
            tok, st = oracle.sample(res["logits"][s][b], p, hist, rng)
            if tok != ids[b][s]:
                assert params.temperature > 0 and \
                    min(st["topp_margin"], st["cdf_margin"]) <= BOUNDARY, (b, s, ids[b][s], tok)
                diverged += 1
                break
            hist.append(tok)
    assert diverged <= 1
    table = TokenBytes.from_file(VOCAB)
    for b in range(8):
        raw = b"".join(table.token_bytes(t) for t in ids[b])
        whole = Utf8Stream()
        assert res["texts"][b] == whole.push_bytes(raw) + whole.flush()
        try:
            # valid UTF-8: the stream equals decode() (tokenizer.rs:270-276); an
            # announced sequence that is not UTF-8 drops the bytes it announced,
            # so then the two differ, as in the reference
            assert res["texts"][b] == raw.decode("utf-8")
        except UnicodeDecodeError:
            pass
    assert out.getvalue() == res["texts"][0]
    print(f"[generate] seed={seed:#x} diverged_at_boundary={diverged} text0={res['texts'][0]!r}",
          flush=True)
