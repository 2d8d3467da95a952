"""Generated ids -> text -> diarised segments, on the host.

* ``decode`` follows ``PromptBuilder::decode`` (prompt.rs:152-155): the
  checkpoint's ``tokenizer.json`` through the ``tokenizers`` library with
  special tokens dropped.
* ``parse`` / ``to_srt`` follow transcript.rs:21-143: the model writes
  ``[start][Sxx]text[end]`` runs; markers are lexed out of the text, a segment
  is (number, speaker, text, number), and anything malformed is skipped rather
  than failing the request.

Numbers are recognised with the grammar of Rust's ``f64::from_str`` (an
optional sign, then ``inf``/``infinity``/``nan`` in any case, or decimal digits
with an optional fraction and exponent), not Python's ``float()``, which also
takes underscores and surrounding whitespace.  SRT milliseconds round half
away from zero like ``f64::round``.
"""
from __future__ import annotations

import math
import re
from dataclasses import dataclass

# char::is_whitespace (Unicode White_Space), what str::trim strips; Python's
# str.strip() also strips U+001C..U+001F.
_WS = ("\t\n\x0b\x0c\r \x85\xa0\u1680\u2000\u2001\u2002\u2003\u2004\u2005\u2006"
       "\u2007\u2008\u2009\u200a\u2028\u2029\u202f\u205f\u3000")


def _trim(s: str) -> str:
    return s.strip(_WS)


_F64 = re.compile(
    r"[+-]?(?:(?:inf|infinity|nan)|(?:\d+\.?\d*|\.\d+)(?:[eE][+-]?\d+)?)\Z", re.IGNORECASE)


@dataclass(frozen=True)
class Segment:
    """One diarised utterance (transcript.rs:5-12)."""

    start: float
    end: float
    speaker: str
    text: str


def _number(s: str) -> float | None:
    """``s.parse::<f64>()`` or None."""
    return float(s) if _F64.match(s) else None


def is_speaker(inner: str) -> bool:
    """``S01``, ``S12``, ``SPEAKER_03`` and similar (transcript.rs:104-112)."""
    s = _trim(inner)
    return (bool(s) and s[0] in "Ss"
            and all((c.isascii() and c.isalnum()) or c == "_" for c in s[1:])
            and any(c.isascii() and c.isdigit() for c in s))


def _lex(text: str) -> list[tuple[str, object]]:
    """Bracketed markers and the free text between them (transcript.rs:67-101)."""
    tokens: list[tuple[str, object]] = []
    rest = text
    while True:
        open_ = rest.find("[")
        if open_ < 0:
            break
        before = rest[:open_]
        if _trim(before):
            tokens.append(("text", before))
        after_open = rest[open_ + 1:]
        close = after_open.find("]")
        if close < 0:
            if _trim(after_open):
                tokens.append(("text", after_open))
            return tokens
        inner = after_open[:close]
        n = _number(_trim(inner))
        if n is not None:
            tokens.append(("number", n))
        elif is_speaker(inner):
            tokens.append(("speaker", _trim(inner)))
        else:
            tokens.append(("text", f"[{inner}]"))
        rest = after_open[close + 1:]
    if _trim(rest):
        tokens.append(("text", rest))
    return tokens


def parse(text: str) -> list[Segment]:
    """Segments of a raw transcript (transcript.rs:21-58)."""
    tokens = _lex(text)
    out: list[Segment] = []
    i = 0
    while i < len(tokens):
        kinds = [t[0] for t in tokens[i:i + 4]]
        if kinds != ["number", "speaker", "text", "number"]:
            i += 1
            continue
        body = _trim(tokens[i + 2][1])
        if body:
            out.append(Segment(tokens[i][1], tokens[i + 3][1], tokens[i + 1][1], body))
        i += 4
    return out


def srt_time(seconds: float) -> str:
    """``HH:MM:SS,mmm`` (transcript.rs:131-143)."""
    s = 0.0 if math.isnan(seconds) else max(seconds, 0.0)
    # f64::round (half away from zero), then `as u64`, which saturates
    total_ms = min(int(math.floor(s * 1000.0 + 0.5)), 2 ** 64 - 1) if math.isfinite(s) else 2 ** 64 - 1
    ms, total_s = total_ms % 1000, total_ms // 1000
    return f"{total_s // 3600:02d}:{(total_s % 3600) // 60:02d}:{total_s % 60:02d},{ms:03d}"


def to_srt(segments: list[Segment], show_speaker: bool) -> str:
    """SRT numbered from one (transcript.rs:114-129)."""
    out = []
    for i, seg in enumerate(segments):
        out.append(f"{i + 1}\n{srt_time(seg.start)} --> {srt_time(seg.end)}\n")
        if show_speaker:
            out.append(f"{seg.speaker}: ")
        out.append(seg.text)
        out.append("\n\n")
    return "".join(out)


def decode(tokenizer, ids) -> str:
    """Generated ids to text without special tokens (prompt.rs:152-155).
    ``tokenizer`` is a ``tokenizers.Tokenizer`` or the path of a
    ``tokenizer.json``."""
    if isinstance(tokenizer, str) or hasattr(tokenizer, "__fspath__"):
        from tokenizers import Tokenizer

        tokenizer = Tokenizer.from_file(str(tokenizer))
    return tokenizer.decode([int(i) for i in ids], skip_special_tokens=True)
