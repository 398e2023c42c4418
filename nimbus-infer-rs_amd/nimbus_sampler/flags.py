"""The `generate` flag surface of the reference CLI, mirrored on the host.

The reference parses `nimbus-rs generate` options into SamplingParams
(src/main.rs:147-155) with its own flag reader (main.rs:65-125):

  --name value   when the next argument exists and does not start with "--";
  --name         otherwise (an empty value: a present switch);
  anything else  a positional argument.

Numbers use Rust's `str::parse`: `f32_of` parses a decimal straight to the
nearest f32 (ties to even), `usize_of` takes an optional '+' and decimal
digits.  An unset or unparsable `--seed` becomes None, which the decode loop
turns into 0x5DEECE66D (engine.rs:271), although the help text says 0.
"""
import dataclasses
import fractions
import re
from typing import Dict, List, Optional, Tuple

import numpy as np

DEFAULT_SEED = 0x5DEECE66D  # engine.rs:271

# ASCII digits only, matched over the whole text (a trailing newline or a
# non-ASCII digit is a bad number, as for Rust's str::parse)
_FLOAT_RE = re.compile(r"[+-]?(?:(\d+\.?\d*|\.\d+)([eE][+-]?\d+)?)", re.ASCII)
_SPECIAL_RE = re.compile(r"([+-]?)(inf|infinity|nan)", re.IGNORECASE | re.ASCII)
_UINT_RE = re.compile(r"\+?\d+", re.ASCII)


class FlagError(ValueError):
    pass


def parse_f32(text: str) -> np.float32:
    """Rust's `f32::from_str`: the decimal rounded once, to nearest, ties to
    even; "inf", "infinity" and "nan" in any case, with an optional sign."""
    m = _SPECIAL_RE.fullmatch(text)
    if m:
        sign = -1.0 if m.group(1) == "-" else 1.0
        return np.float32(np.nan) if m.group(2).lower() == "nan" else np.float32(sign * np.inf)
    if not _FLOAT_RE.fullmatch(text):
        raise FlagError(f"bad number {text!r}")
    exact = fractions.Fraction(text)
    mag = abs(exact)
    # the f32 neighbours of the f64 nearest, then the exact nearest of those
    fmax = np.finfo(np.float32).max
    f = np.float32(float(mag)) if mag <= fractions.Fraction(float(fmax)) else fmax
    with np.errstate(over="ignore"):
        cands = {f, np.nextafter(f, np.float32(0)), np.nextafter(f, np.float32(np.inf))}
    best = None
    for c in sorted(cands):
        if not np.isfinite(c):
            continue
        d = abs(fractions.Fraction(float(c)) - mag)
        key = (d, int(np.frombuffer(np.float32(c).tobytes(), np.uint32)[0]) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    r = best[1]
    # overflow: at or beyond the midpoint between FLT_MAX and 2^128
    if mag >= fractions.Fraction(float(fmax)) + fractions.Fraction(2) ** 103:
        r = np.float32(np.inf)
    return np.float32(-r) if exact < 0 or text.startswith("-") else np.float32(r)


def parse_uint(text: str, bits: int = 64) -> int:
    """Rust's `usize` / `u64` `from_str`: optional '+', decimal digits, in range."""
    if not _UINT_RE.fullmatch(text):
        raise FlagError(f"bad number {text!r}")
    v = int(text.lstrip("+"))
    if v >= 1 << bits:
        raise FlagError(f"bad number {text!r}")
    return v


@dataclasses.dataclass
class Flags:
    """main.rs:65-125: `--name value` pairs, switches and positionals."""
    map: Dict[str, str]
    positional: List[str]

    @classmethod
    def parse(cls, args: List[str]) -> "Flags":
        m: Dict[str, str] = {}
        pos: List[str] = []
        i = 0
        while i < len(args):
            a = args[i]
            if a.startswith("--"):
                name = a[2:]
                if i + 1 < len(args) and not args[i + 1].startswith("--"):
                    m[name] = args[i + 1]
                    i += 2
                else:
                    m[name] = ""
                    i += 1
            else:
                pos.append(a)
                i += 1
        return cls(m, pos)

    def get(self, name: str) -> Optional[str]:
        return self.map.get(name)

    def has(self, name: str) -> bool:
        return name in self.map

    def require(self, name: str) -> str:
        v = self.get(name)
        if v is None:
            raise FlagError(f"missing required flag --{name}")
        return v

    def usize_of(self, name: str, default: int) -> int:
        v = self.get(name)
        if v is None:
            return default
        try:
            return parse_uint(v)
        except FlagError:
            raise FlagError(f"--{name}: bad number {v!r}") from None

    def f32_of(self, name: str, default: float) -> np.float32:
        v = self.get(name)
        if v is None:
            return np.float32(default)
        try:
            return parse_f32(v)
        except FlagError:
            raise FlagError(f"--{name}: bad number {v!r}") from None


def generate_params(args: List[str]):
    """cmd_generate's SamplingParams (main.rs:147-155) and the seed the decode
    loop uses (engine.rs:271).  Returns (SamplingParams, rng seed, Flags)."""
    from . import SamplingParams
    flags = Flags.parse(args)
    seed_text = flags.get("seed")
    seed: Optional[int] = None
    if seed_text is not None:
        try:
            seed = parse_uint(seed_text)
        except FlagError:
            seed = None  # `.and_then(|s| s.parse().ok())`: an unparsable seed is unset
    params = SamplingParams(
        max_new_tokens=flags.usize_of("max-new-tokens", 64),
        temperature=float(flags.f32_of("temperature", 0.0)),
        top_k=flags.usize_of("top-k", 0),
        top_p=float(flags.f32_of("top-p", 1.0)),
        repetition_penalty=float(flags.f32_of("repetition-penalty", 1.0)),
        seed=seed,
        stop_tokens=[],
    )
    return params, (seed if seed is not None else DEFAULT_SEED), flags
