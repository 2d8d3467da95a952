"""Transcript parsing and SRT export: the reference's own cases
(transcript.rs:145-227) as vectors, plus the places where Rust's semantics
differ from Python's defaults (f64 grammar, str::trim, f64::round)."""
import importlib

import pytest

tr = importlib.import_module("fast-moss-diarization_amd.transcript")
Seg = tr.Segment


# transcript.rs:149-166
def test_documented_format():
    segs = tr.parse("[0.48][S01]Welcome everyone[1.66][12.26][S02]Ready for evaluation[13.81]")
    assert segs == [Seg(0.48, 1.66, "S01", "Welcome everyone"),
                    Seg(12.26, 13.81, "S02", "Ready for evaluation")]


# transcript.rs:168-173
def test_portuguese_text_intact():
    assert tr.parse("[3.64][S01] e dar aqui a sua opinião.[5.52]") == [
        Seg(3.64, 5.52, "S01", "e dar aqui a sua opinião.")]


# transcript.rs:175-181, 183-188, 190-195, 197-201
@pytest.mark.parametrize("text,texts", [
    ("[0.0][S01]complete[1.0][2.0][S02]cut off here", ["complete"]),
    ("garbage [S01]no start time[1.0] [5.0][S02]good[6.0]", ["good"]),
    ("", []),
    ("   \n ", []),
    ("[0.0][S01]   [1.0]", []),
    ("[0.0][S01]fine[1.0][2.0", ["fine"]),
])
def test_partial_and_malformed(text, texts):
    assert [s.text for s in tr.parse(text)] == texts


# transcript.rs:203-211
@pytest.mark.parametrize("inner,want", [
    ("S01", True), ("S1", True), ("SPEAKER_03", True), ("s7", True), (" S02 ", True),
    ("Speaker", False), ("1.5", False), ("", False), ("S0-1", False), ("S١", False),
])
def test_speaker_detection(inner, want):
    assert tr.is_speaker(inner) is want


# transcript.rs:213-218, plus f64::round's half-away-from-zero and saturation
@pytest.mark.parametrize("sec,want", [
    (0.0, "00:00:00,000"), (1.5, "00:00:01,500"), (3661.25, "01:01:01,250"),
    (0.0005, "00:00:00,001"), (0.0025, "00:00:00,003"), (-3.0, "00:00:00,000"),
    (float("nan"), "00:00:00,000"),
])
def test_srt_time(sec, want):
    assert tr.srt_time(sec) == want


# transcript.rs:220-226
def test_srt_numbers_from_one():
    segs = tr.parse("[0.0][S01]one[1.0][1.0][S02]two[2.0]")
    srt = tr.to_srt(segs, True)
    assert srt.startswith("1\n00:00:00,000 --> 00:00:01,000\nS01: one\n\n2\n")
    assert "S01:" not in tr.to_srt(segs, False)
    assert srt == ("1\n00:00:00,000 --> 00:00:01,000\nS01: one\n\n"
                   "2\n00:00:01,000 --> 00:00:02,000\nS02: two\n\n")


# markers are numbers only under Rust's f64 grammar
@pytest.mark.parametrize("marker,is_number", [
    ("1.5", True), ("+1.5", True), (" 2.0 ", True), ("1e3", True), ("1.", True), (".5", True),
    ("1.e2", True), ("inf", True), ("-Infinity", True), ("NaN", True),
    ("1_0", False), ("e5", False), ("1e", False), (".", False), ("0x10", False), ("", False),
])
def test_number_markers(marker, is_number):
    segs = tr.parse(f"[{marker}][S01]x[9.0]")
    assert (len(segs) == 1) is is_number
    if not is_number:
        # an unrecognised marker stays in the text as literal brackets
        assert tr._lex(f"[{marker}]") == [("text", f"[{marker}]")]


def test_trim_is_rusts():
    # U+001C is whitespace to Python's strip() but not to str::trim: the body
    # "\x1c" is kept, so the segment survives
    assert [s.text for s in tr.parse("[0.0][S01]\x1c[1.0]")] == ["\x1c"]
    # U+3000 (ideographic space) is whitespace to both
    assert tr.parse("[0.0][S01]　[1.0]") == []


def test_decode_drops_special_tokens(tmp_path):
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import models, pre_tokenizers, decoders

    vocab = {"<|im_end|>": 0, "hello": 1, "world": 2, "[0.5]": 3}
    tok = tokenizers.Tokenizer(models.WordLevel(vocab, unk_token="hello"))
    tok.pre_tokenizer = pre_tokenizers.Whitespace()
    tok.decoder = decoders.WordPiece()
    tok.add_special_tokens(["<|im_end|>"])
    path = tmp_path / "tokenizer.json"
    tok.save(str(path))
    assert tr.decode(str(path), [1, 2, 0]) == "hello world"
    assert tr.decode(tok, [0, 1]) == "hello"
