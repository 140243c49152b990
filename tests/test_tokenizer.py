"""Tekken tokenizer and chat framing on the CPU (lunelette_amd/csrc/tokenizer.c,
chat.c).

Oracles:
- the reference's tokenizer, JSON reader and chat framing built from
  src/tokenizer.c, src/tokenizer_json.c and src/chat.c into
  oracle/_ref/libreftok.so: every case below that has a verdict or ids is
  also run through it and must agree;
- the `regex` package applying the pre-tokenizer pattern itself: piece
  boundaries of random multilingual text must equal regex.finditer's;
- a direct restatement of byte-pair merging (lowest rank, leftmost tie) as
  in tests/test_tokenizer_bpe.c:31-63, exhaustive over a/b strings.
Cases restated from tests/test_tokenizer.c:21-74 (JSON grammar and limits),
:78-95 and :98-201 (round trips, limits, invalid UTF-8 and ids, the fixture's
merges), tests/test_tokenizer.c:262-279 (defective files) and
tests/test_chat.c:27-61. Allocation failure (tests/test_tokenizer_alloc.c)
through the test library's host allocation seam, at every allocation of open,
encode (32768 bytes), decode and chat framing rather than the first three.
"""
import ctypes
import os
import random

import numpy as np

import pytest
import regex

import lunelette_amd as lh
from lunelette_amd.tokenizer import LONG_INPUT, Tokenizer, split
from tokenizer_files import (PATTERN, ranks_with_tokens, synthetic_ranks, write_tekken)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REFTOK = os.path.join(ROOT, "oracle", "_ref", "libreftok.so")


@pytest.fixture(scope="module")
def product_lib(product):
    return product


@pytest.fixture(scope="module")
def libraries(product_lib):
    """The product, and the reference build when it exists."""
    libs = [("product", product_lib)]
    if os.path.exists(REFTOK):
        ref = ctypes.CDLL(REFTOK)
        lh.declare_tokenizer(ref)
        libs.append(("reference", ref))
    return libs


@pytest.fixture(scope="module")
def synthetic(tmp_path_factory):
    path = tmp_path_factory.mktemp("tok") / "synthetic.json"
    write_tekken(path, synthetic_ranks())
    return path


def opens(path, library):
    try:
        Tokenizer(path, library).close()
        return True
    except ValueError:
        return False


def test_defective_files_rejected(tmp_path, libraries):
    """tests/test_tokenizer.c:262-268 with tests/support/tokenizer_fixture.h:32-99."""
    for defect in range(1, 12):
        path = tmp_path / ("defect%d.json" % defect)
        write_tekken(path, synthetic_ranks(defect), defect)
        for name, library in libraries:
            assert not opens(path, library), (name, defect)
        os.remove(path)
    for field, value in (("version", "v12"), ("pattern", PATTERN + "|x"),
                         ("num_vocab_tokens", 131071), ("default_num_special_tokens", 999)):
        path = tmp_path / "config.json"
        write_tekken(path, synthetic_ranks(), config={field: value})
        for name, library in libraries:
            assert not opens(path, library), (name, field)
        os.remove(path)


JSON_ACCEPTED = [
    '"\\u0000\\u00e9\\u20ac\\uD83D\\uDE00"', "4294967295", "[true,false,null,-0.5e+3,{},[]]",
    "[" * 32 + "]" * 32, '"' + "x" * 4096 + '"',
    "{" + ",".join('"k%d":0' % i for i in range(64)) + "}", "1" * 128, "-0", "1E-9",
    '"\\"\\\\\\/\\b\\f\\n\\r\\t"', ' \t\r\n[ 1 , 2 ]\n',
]
JSON_REJECTED = [
    "{", "[1,]", '{"a":1,}', '{"a":1,"a":2}', '{"a":1,"\\u0061":2}', "[01]", "[-]", "[1.]",
    "[1e+]", "[true false]", '"\\uD800"', '"\\uDC00"', '"\\x"', b'"\xc0\x80"', b'"\xed\xa0\x80"',
    b'"\xf4\x90\x80\x80"', '"\n"', "[" * 33 + "]" * 33, '"' + "x" * 4097 + '"',
    "{" + ",".join('"k%d":0' % i for i in range(65)) + "}", "1" * 129, "nul", "tru", "+1",
    "'a'", '"\\u12"', '{"a" 1}', "[1 2]", "", "01",
]


def test_json_reader_grammar_and_limits(tmp_path, libraries):
    """tests/test_tokenizer.c:21-74: each construct sits in an extra root
    member of a valid file, so the verdict is the JSON reader's."""
    ranks = synthetic_ranks()
    for k, extra in enumerate(JSON_ACCEPTED + JSON_REJECTED):
        want = k < len(JSON_ACCEPTED)
        path = tmp_path / ("json%d.json" % k)
        write_tekken(path, ranks, extra=extra)
        for name, library in libraries:
            assert opens(path, library) == want, (name, extra[:40])
        os.remove(path)
    path = tmp_path / "trailing.json"
    write_tekken(path, ranks)
    with open(path, "ab") as f:
        f.write(b" x")
    for name, library in libraries:
        assert not opens(path, library), name


def roundtrip(t, text):
    ids = t.encode(text)
    assert all(1000 <= i < 131072 for i in ids)
    assert t.decode(ids) == text
    return ids


def contract(t, synthetic_file):
    """tests/test_tokenizer.c:78-201."""
    roundtrip(t, b"")
    for text in ["Hello world!", "[INST]<s></s>[/INST][SYSTEM_PROMPT]", "aaa aaaa aaaaa",
                 "CamelCase HTTPServer 12345\r\n\t  !/\n",
                 "日本語 Ελληνικά مرحبا 😀 é\x1c\xa0"]:
        roundtrip(t, text.encode())
    roundtrip(t, bytes(range(128)))
    roundtrip(t, b"a" * 4096)
    with pytest.raises(ValueError):
        t.encode(b"a" * 4097)
    long_text = b"7" * 32769
    for size in (0, 4096, 4097, 32768):
        ids = t.encode(long_text[:size], LONG_INPUT)
        assert len(ids) == size
        if synthetic_file:
            assert all(i == 1000 + ord("7") for i in ids)
    for size, limit in ((32769, 32768), (1, 4097), (4097, 4096), (1, 2 ** 64 - 1)):
        with pytest.raises(ValueError):
            t.encode(long_text[:size], limit)
    with pytest.raises(ValueError, match="invalid UTF-8 at byte 32767"):
        t.encode(long_text[:32767] + b"\x80", LONG_INPUT)
    for bad in (b"\x80", b"\xc0\x80", b"\xed\xa0\x80", b"\xf4\x90\x80\x80", b"\xe2\x82"):
        with pytest.raises(ValueError):
            t.encode(bad)
    for bad in (0, 999, 131072, 0xFFFFFFFF):
        with pytest.raises(ValueError):
            t.decode([bad])
    with pytest.raises(ValueError):
        t.decode([1000] * 4097)
    with pytest.raises(ValueError):
        t.decode([1000, 1001, 2])
    assert t.decode([]) == b""
    if synthetic_file:
        assert t.encode(b"aaaa") == [1256, 1256]
        assert t.encode(b"aaa") == [1257]
        assert t.encode(b"aaaaa") == [1256, 1257]
        assert t.encode(b"aA") == [1097, 1065]
        raw = [1000 + 0xF0, 1000 + 0x9F, 1000 + 0x98, 1000 + 0x80, 1000, 1255]
        assert t.decode(raw) == b"\xf0\x9f\x98\x80\0\xff"


def test_contract_synthetic(synthetic, libraries):
    for name, library in libraries:
        with Tokenizer(synthetic, library) as t:
            contract(t, True)


def legacy_merge(rank_of, piece):
    """Byte-pair merging as tests/test_tokenizer_bpe.c:31-63 states it: the
    whole piece if it is a token, else repeatedly merge the adjacent pair of
    lowest rank (leftmost on equal ranks) until none is a token."""
    if piece in rank_of:
        return [rank_of[piece] + 1000]
    parts = [piece[i:i + 1] for i in range(len(piece))]
    while len(parts) > 1:
        best = None
        for i in range(len(parts) - 1):
            r = rank_of.get(parts[i] + parts[i + 1])
            if r is not None and (best is None or r < best[0]):
                best = (r, i)
        if best is None:
            break
        i = best[1]
        parts[i:i + 2] = [parts[i] + parts[i + 1]]
    return [rank_of[p] + 1000 for p in parts]


SMALL = [b"a", b"b", b"aa", b"ab", b"ba", b"bb", b"aaa", b"aab", b"abba", b"aaaa", b" "]


def ab_strings(n):
    for bits in range(1 << n):
        yield b"".join(b"a" if (bits >> i) & 1 else b"b" for i in range(n))


def test_merges_exhaustive(tmp_path, libraries):
    """tests/test_tokenizer_bpe.c:65-120: every a/b string up to 12 bytes with
    the frozen ranks, then up to 8 bytes under 6 shuffled rank orders."""
    rng = random.Random(72619)
    orders = [list(range(len(SMALL)))]
    for _ in range(6):
        order = list(range(len(SMALL)))
        rng.shuffle(order)
        orders.append(order)
    for k, order in enumerate(orders):
        tokens = [None] * len(SMALL)
        for i, r in enumerate(order):
            tokens[r] = SMALL[i]
        ranks = ranks_with_tokens(tokens)
        rank_of = {b: r for r, b in enumerate(ranks)}
        path = tmp_path / ("small%d.json" % k)
        write_tekken(path, ranks)
        opened = [(name, Tokenizer(path, library)) for name, library in libraries]
        for n in range(1, (12 if k == 0 else 8) + 1):
            for text in ab_strings(n):
                want = legacy_merge(rank_of, text)
                for name, t in opened:
                    assert t.encode(text) == want, (name, text, order)
        for _, t in opened:
            t.close()
        os.remove(path)


POOL = ("aAbBzZ eé Éß ΣσΩ жЖ 日本 ٠١مر ב 한글 ǅ ʰ ̀ ́ ﬁ Ⅻ ½ ² 0 7 9 , . ! ? / \\ - _ ( ) [ ] "
        "😀 👍🏽 € $ @ # ' \" \t \r \n \x0b \x0c \x85 \xa0   　 \x1c \x01 ~ ^ `").split(" ")
POOL += [" ", "  ", "\r\n", "\n\n", " \n", "\t\n "]


def random_texts(seed, count, max_len):
    rng = random.Random(seed)
    for _ in range(count):
        yield "".join(rng.choice(POOL) for _ in range(rng.randrange(max_len + 1)))


def test_pieces_match_regex(product_lib):
    """Piece ends of the product's splitter equal regex.finditer's."""
    engine = regex.compile(PATTERN)
    for text in list(random_texts(5, 3000, 24)) + ["", " ", "  a", "a  ", "\r\n\r\n x",
                                                     "  \n  ", "a/\n", " !/\r\nx"]:
        data = text.encode()
        want = [len(text[:m.end()].encode()) for m in engine.finditer(text)]
        assert split(data, product_lib) == want, repr(text)


def rich_ranks():
    """Ranks where merges cross every kind of piece boundary: all pairs and
    some triples over a small alphabet, and the UTF-8 of a few letters."""
    alphabet = [b"a", b"b", b"e", b"A", b"Z", b" ", b"\n", b"\r", b"7", b",", b"!", b"/", b"\t"]
    tokens = []
    for x in alphabet:
        for y in alphabet:
            tokens.append(x + y)
    for x in alphabet[:6]:
        for y in alphabet[:6]:
            for z in alphabet[:4]:
                tokens.append(x + y + z)
    for ch in "éÉσΣжЖ日本😀":
        tokens.append(ch.encode())
    tokens += [b" \xc3", b"\xc3\xa9a", b"  \n", b"aaaa", b"\n\n\n"]
    seen, unique = set(), []
    for tok in tokens:
        if tok not in seen:
            seen.add(tok)
            unique.append(tok)
    rng = random.Random(11)
    rng.shuffle(unique)
    return ranks_with_tokens(unique)


def test_encode_matches_reference_and_restatement(tmp_path, libraries):
    ranks = rich_ranks()
    rank_of = {b: r for r, b in enumerate(ranks)}
    path = tmp_path / "rich.json"
    write_tekken(path, ranks)
    engine = regex.compile(PATTERN)
    opened = [(name, Tokenizer(path, library)) for name, library in libraries]
    alphabet = ["a", "b", "e", "A", "Z", " ", "\n", "\r", "7", ",", "!", "/", "\t", "é", "É",
                "σ", "Σ", "ж", "Ж", "日", "本", "😀", "  ", "\r\n"]
    rng = random.Random(3)
    texts = ["".join(rng.choice(alphabet) for _ in range(rng.randrange(40))) for _ in range(3000)]
    texts += list(random_texts(9, 500, 30))
    for text in texts:
        want = []
        for m in engine.finditer(text):
            want += legacy_merge(rank_of, m.group().encode())
        for name, t in opened:
            assert t.encode(text) == want, (name, repr(text))
            assert t.decode(want) == text.encode()
    for _, t in opened:
        t.close()


def test_chat_framing(synthetic, libraries):
    """tests/test_chat.c:27-61 (single bytes are ids 1000 + byte in the fixture)."""
    for name, library in libraries:
        with Tokenizer(synthetic, library) as t:
            assert t.chat_prompt("u", "s") == (0, [1, 17, 1115, 18, 3, 1117, 4])
            assert t.chat_prompt("") == (0, [1, 3, 4])
            assert t.chat_prompt("", "") == (0, [1, 17, 18, 3, 4])
            assert t.chat_prompt("x", raw=True) == (0, [1, 1120])
            assert t.chat_prompt("x", "", raw=True)[0] == -1
            status, ids = t.chat_prompt("x" * 255, raw=True)
            assert status == 0 and len(ids) == 256
            assert t.chat_prompt("x" * 255)[0] == -1          # 258 ids do not fit
            assert t.chat_prompt(b"\xff")[0] == -1
            assert t.chat_prompt("u", b"\xff")[0] == -1


REFERENCE_TABLE = "/root/reference/src/tokenizer_unicode.h"


def shipped_classes():
    import re as _re
    text = open(os.path.join(ROOT, "lunelette_amd", "csrc", "lh_unicode_classes.h")).read()
    table = bytearray(0x110000)
    for a, b, m in _re.findall(r"\{0x([0-9a-f]+), 0x([0-9a-f]+), (\d+)\}", text):
        table[int(a, 16):int(b, 16) + 1] = bytes([int(m)]) * (int(b, 16) - int(a, 16) + 1)
    return table


def test_class_table_matches_reference_table():
    """Every code point has the class the reference tokenizer's generated
    property table (Unicode 18.0.0) gives it, mapped onto the pattern's five
    classes."""
    if not os.path.exists(REFERENCE_TABLE):
        pytest.skip("the reference checkout is not present")
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "gen", os.path.join(ROOT, "lunelette_amd", "csrc", "gen_unicode_classes.py"))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    ranges, version = gen.reference_ranges(REFERENCE_TABLE)
    assert "Unicode 18" in version
    want = bytearray(0x110000)
    for a, b, m in ranges:
        want[a:b + 1] = bytes([gen.from_reference_mask(m)]) * (b - a + 1)
    assert shipped_classes() == want


# Code points whose class Unicode 18 assigns and the installed regex package's
# older data does not (letters, numbers, marks), mixed with ASCII.
UNICODE18 = ["\U0003d000", "\U0003d5a1", "\U00018e00", "\U00019191", "\U00012550",
             "\U00012686"]


def test_unicode18_text_matches_reference_tokenizer(tmp_path, libraries):
    if len(libraries) < 2:
        pytest.skip("oracle/_ref/libreftok.so not built")
    table = shipped_classes()
    assert all(table[ord(c)] for c in UNICODE18)
    path = tmp_path / "rich18.json"
    write_tekken(path, rich_ranks())
    opened = [(name, Tokenizer(path, library)) for name, library in libraries]
    alphabet = UNICODE18 + ["a", "Z", " ", "7", "\n", "é", "日", "!", "'s"]
    rng = random.Random(18)
    texts = ["".join(rng.choice(alphabet) for _ in range(rng.randrange(1, 30)))
             for _ in range(2000)]
    engine = regex.compile(PATTERN)
    boundaries_differ = 0
    for text in texts:
        ids = [t.encode(text) for _, t in opened]
        assert ids[0] == ids[1], repr(text)
        ends, at = [], 0
        for m in engine.finditer(text):
            at += len(m.group().encode())
            ends.append(at)
        boundaries_differ += ends != split(text)
    # The texts exercise the new assignments: the installed regex (older
    # Unicode data) splits many of them differently.
    assert boundaries_differ > 100
    for _, t in opened:
        t.close()


def each_allocation_failure(seams, attempt):
    """Runs attempt() with the nth host allocation failing, n = 1, 2, ...,
    until one run allocates no more than n - 1 times and succeeds. Every
    failing run must free all it allocated. Returns the successful result and
    the number of allocations it made."""
    base = seams.lunelette_metal_test_live_host_allocations()
    nth = 1
    while True:
        assert nth < 100000, "no run succeeded"
        seams.lunelette_metal_test_fail_host_allocation(nth)
        try:
            result = attempt()
        except ValueError as e:
            assert "out of memory" in str(e), (nth, str(e))
            assert seams.lunelette_metal_test_live_host_allocations() == base, nth
            nth += 1
            continue
        finally:
            made = seams.lunelette_metal_test_host_allocations()
        seams.lunelette_metal_test_fail_host_allocation(0)
        assert made == nth - 1, (made, nth)
        return result, made


def test_allocation_failures_clean_up(synthetic, libraries):
    seams = lh.test_lib()
    lh.declare_tokenizer(seams)
    reference = dict(libraries).get("reference")
    try:
        tok, made = each_allocation_failure(seams, lambda: Tokenizer(synthetic, seams))
        assert made >= 4
        live = seams.lunelette_metal_test_live_host_allocations()
        text = b"a" * LONG_INPUT    # the reference test's input
        ids, made = each_allocation_failure(seams, lambda: tok.encode(text, limit=LONG_INPUT))
        assert made >= 3
        # The returned ids are counted until the caller frees them (with free).
        assert seams.lunelette_metal_test_live_host_allocations() == live + 1
        if reference is not None:
            with Tokenizer(synthetic, reference) as ref:
                assert ids == ref.encode(text, limit=LONG_INPUT)
        mixed = "Grüße, 東京 — ok?\n\t 12345 " * 40
        ids, _ = each_allocation_failure(seams, lambda: tok.encode(mixed))
        raw, _ = each_allocation_failure(seams, lambda: tok.decode(ids))
        assert raw == mixed.encode()
        framed, _ = each_allocation_failure(seams, lambda: chat(seams, tok, mixed[:60]))
        assert framed[0] == 1 and len(framed) > 20
        with pytest.raises(ValueError, match="invalid UTF-8 at byte %d" % (LONG_INPUT - 1)):
            tok.encode(text[:-1] + b"\x80", limit=LONG_INPUT)
        tok.close()
    finally:
        seams.lunelette_metal_test_fail_host_allocation(0)


def chat(library, tok, prompt):
    """Ids of lunelette_chat_prompt; ValueError with its diagnostic."""
    ids = np.full(256, -7, np.int64)
    count = ctypes.c_size_t(999)
    err = ctypes.create_string_buffer(512)
    if library.lunelette_chat_prompt(tok.handle, prompt.encode(), None, 0,
                                     ids.ctypes.data_as(lh.c_int64_p), ctypes.byref(count),
                                     err, 512):
        assert count.value == 999 and np.all(ids == -7)
        raise ValueError(err.value.decode())
    return ids[:count.value].tolist()
