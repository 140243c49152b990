"""Tekken13 tokenizer files for the tests (test infrastructure).

write_tekken() writes the supported schema: config v13 with the canonical
pre-tokenizer pattern, 130072 ordinary ranks as canonical base64 and 1000
special tokens with the framing spellings. synthetic_ranks() gives the small
fixture the reference's tests use (tests/support/tokenizer_fixture.h:32-99):
single bytes at ranks 0..255, "aa" 256, "aaa" 257, "aA" 258, and unique
5-byte fillers; the defects 1..11 are the same broken variants.
"""
import base64
import json

PATTERN = (r"[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]*[\p{Ll}\p{Lm}\p{Lo}\p{M}]+|"
           r"[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]+[\p{Ll}\p{Lm}\p{Lo}\p{M}]*|"
           r"\p{N}| ?[^\s\p{L}\p{N}]+[\r\n/]*|\s*[\r\n]+|\s+(?!\S)|\s+")
ORDINARY = 130072
FRAMING = {1: "<s>", 2: "</s>", 3: "[INST]", 4: "[/INST]", 17: "[SYSTEM_PROMPT]",
           18: "[/SYSTEM_PROMPT]"}


def filler(rank):
    return bytes([255, rank & 255, (rank >> 8) & 255, (rank >> 16) & 255, 255])


def synthetic_ranks(defect=0):
    ranks = []
    for rank in range(ORDINARY):
        if rank < 256:
            b = bytes([rank])
        elif rank in (256, 257):
            b = b"a" * (rank - 254)
        elif rank == 258:
            b = b"\0" if defect == 1 else b"aA"
        else:
            b = filler(rank)
        ranks.append(b)
    return ranks


def ranks_with_tokens(tokens):
    """tokens (byte strings) at ranks 0.., then every missing single byte,
    then fillers up to 130072 ranks."""
    ranks = list(tokens)
    present = set(ranks)
    ranks += [bytes([b]) for b in range(256) if bytes([b]) not in present]
    ranks += [filler(r) for r in range(len(ranks), ORDINARY)]
    assert len(set(ranks)) == len(ranks) == ORDINARY
    return ranks


def write_tekken(path, ranks, defect=0, extra=None, config=None):
    """ranks[r] = bytes of ordinary rank r. extra: raw JSON text (str or
    bytes) added as one more root member ("extra"), ignored by the
    tokenizer."""
    cfg = {"pattern": PATTERN, "version": "v13", "num_vocab_tokens": 131072,
           "default_vocab_size": 131072, "default_num_special_tokens": 1000}
    cfg.update(config or {})
    parts = ['{"config":', json.dumps(cfg), ',"vocab":[']
    entries = []
    count = ORDINARY - 1 if defect == 9 else ORDINARY
    for rank in range(count):
        shown = 257 if (rank == 258 and defect == 2) else \
            ORDINARY if (rank == 258 and defect == 5) else rank
        if rank == 258 and defect in (3, 6, 7, 8):
            encoded = {3: "AB==", 6: "", 7: "@@==", 8: "AA=A"}[defect]
        else:
            encoded = base64.b64encode(ranks[rank]).decode()
        entries.append('{"rank":%d,"token_bytes":"%s"}' % (shown, encoded))
    parts.append(",".join(entries))
    parts.append('],"special_tokens":[')
    specials = []
    for rank in range(999 if defect == 11 else 1000):
        shown = 998 if (defect == 4 and rank == 999) else rank
        text = "<s>" if (defect == 10 and rank == 999) else FRAMING.get(rank, "special_%d" % rank)
        specials.append('{"rank":%d,"is_control":true,"token_str":%s}' % (shown, json.dumps(text)))
    parts.append(",".join(specials))
    parts.append("]")
    body = "".join(parts).encode()
    if extra is not None:
        body += b',"extra":' + (extra.encode() if isinstance(extra, str) else extra)
    with open(path, "wb") as f:
        f.write(body + b"}")
