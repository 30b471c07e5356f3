"""Pure-Python restatement of the reference tokenizer
(examples/llm/model/tokenizer.cpp:70-374), for tests on small vocabularies.

TEST INFRASTRUCTURE ONLY: the checker for libxpose's xp_tokenize /
xp_detokenize, never used by the product. Strings are handled as bytes, as
the reference handles std::string_view; each step follows the cited lines.
"""
from __future__ import annotations

import heapq

SPACE = "▁".encode()
NORMAL, UNKNOWN, CONTROL, USER_DEFINED, UNUSED, BYTE = 1, 2, 3, 4, 5, 6


def utf8_len(c: int) -> int:
    """tokenizer.cpp:20-27."""
    if c < 0x80:
        return 1
    if (c & 0xE0) == 0xC0:
        return 2
    if (c & 0xF0) == 0xE0:
        return 3
    if (c & 0xF8) == 0xF0:
        return 4
    return 1


def scan_byte(s: bytes):
    """sscanf(s, "<0x%02X>") == 1 for a six-byte spelling (tokenizer.cpp:150-156,
    321-324): one or two hex digits after "<0x"."""
    if len(s) != 6 or not s.startswith(b"<0x"):
        return None
    digits = b""
    for ch in s[3:5]:
        if chr(ch) in "0123456789abcdefABCDEF":
            digits += bytes([ch])
        else:
            break
    return int(digits, 16) if digits else None


class Tokenizer:
    def __init__(self, tokens, scores=None, types=None, bos=-1, eos=-1, unk=-1, pad=-1,
                 add_space_prefix=True):
        """Tokenizer::from_gguf + build_indices (tokenizer.cpp:70-165)."""
        self.tokens = [t.encode() if isinstance(t, str) else bytes(t) for t in tokens]
        n = len(self.tokens)
        self.scores = list(scores) if scores is not None else [0.0] * n
        self.types = list(types) if types is not None else [NORMAL] * n
        self.bos, self.eos, self.unk, self.pad = bos, eos, unk, pad
        self.add_space_prefix = add_space_prefix
        self.token_to_id = {}
        special = []
        self.byte_to_id = [-1] * 256
        for i, t in enumerate(self.tokens):
            self.token_to_id.setdefault(t, i)
            if self.types[i] in (CONTROL, UNKNOWN):
                special.append(i)
            if self.types[i] == BYTE and len(t) == 6 and t.startswith(b"<0x") and t[5:6] == b">":
                v = scan_byte(t)
                if v is not None and v < 256:
                    self.byte_to_id[v] = i
        special.sort(key=lambda i: -len(self.tokens[i]))
        self.special_lengths = []
        for i in special:
            ln = len(self.tokens[i])
            if ln and (not self.special_lengths or self.special_lengths[-1] != ln):
                self.special_lengths.append(ln)
        seen = []
        for ln in self.special_lengths:
            if not seen or seen[-1] != ln:
                seen.append(ln)
        self.special_lengths = seen

    def tokenize_fragment(self, raw: bytes, out: list) -> None:
        """tokenizer.cpp:193-297."""
        if not raw:
            return
        norm = (SPACE if self.add_space_prefix else b"") + raw.replace(b" ", SPACE)
        syms = []
        i = 0
        while i < len(norm):
            ln = min(utf8_len(norm[i]), len(norm) - i)
            s = {"prev": len(syms) - 1, "at": i, "n": ln}
            i += ln
            s["next"] = -1 if i == len(norm) else len(syms) + 1
            syms.append(s)
        if not syms:
            return
        work = []           # max-heap on score, then leftmost: (-score, left, right, size)
        rev_merge = {}

        def text(k):
            return norm[syms[k]["at"]:syms[k]["at"] + syms[k]["n"]]

        def try_add(left, right):
            if left == -1 or right == -1:
                return
            t = norm[syms[left]["at"]:syms[left]["at"] + syms[left]["n"] + syms[right]["n"]]
            if t not in self.token_to_id:
                return
            heapq.heappush(work, (-float(self.scores[self.token_to_id[t]]), left, right, len(t)))
            rev_merge[t] = (left, right)

        for k in range(1, len(syms)):
            try_add(k - 1, k)
        while work:
            _, left, right, size = heapq.heappop(work)
            l, r = syms[left], syms[right]
            if l["n"] == 0 or r["n"] == 0 or l["n"] + r["n"] != size:
                continue
            l["n"] += r["n"]
            r["n"] = 0
            l["next"] = r["next"]
            if r["next"] >= 0:
                syms[r["next"]]["prev"] = left
            try_add(l["prev"], left)
            try_add(left, l["next"])

        def emit(k):
            t = text(k)
            if t in self.token_to_id:
                out.append(self.token_to_id[t])
                return
            if t in rev_merge:
                a, b = rev_merge[t]
                emit(a)
                emit(b)
                return
            for byte in t:
                bid = self.byte_to_id[byte]
                if bid >= 0:
                    out.append(bid)
                elif self.unk >= 0:
                    out.append(self.unk)

        k = 0
        while k != -1:
            if syms[k]["n"] > 0:
                emit(k)
            k = syms[k]["next"]

    def encode(self, text: bytes, add_bos: bool = False, add_eos: bool = False) -> list:
        """tokenizer.cpp:299-343."""
        out = []
        if add_bos and self.bos >= 0:
            out.append(self.bos)
        i = frag = 0
        while i < len(text):
            hit = -1
            for ln in self.special_lengths:
                if ln > len(text) - i:
                    continue
                tid = self.token_to_id.get(text[i:i + ln])
                if tid is None:
                    continue
                if self.types[tid] in (CONTROL, UNKNOWN):
                    hit = tid
                    break
            if hit >= 0:
                self.tokenize_fragment(text[frag:i], out)
                out.append(hit)
                i += len(self.tokens[hit])
                frag = i
            else:
                i += 1
        self.tokenize_fragment(text[frag:], out)
        if add_eos and self.eos >= 0:
            out.append(self.eos)
        return out

    def decode_one(self, tid: int) -> bytes:
        """tokenizer.cpp:348-367."""
        s = self.tokens[tid] if 0 <= tid < len(self.tokens) else b""
        ty = self.types[tid] if 0 <= tid < len(self.types) else 0
        if ty == BYTE:
            v = scan_byte(s) if len(s) == 6 else None
            return bytes([v & 0xFF]) if v is not None else s
        return s.replace(SPACE, b" ")

    def decode(self, ids, skip_special: bool = True) -> bytes:
        """tokenizer.cpp:351-374."""
        out = b""
        first = True
        for tid in ids:
            ty = self.types[tid] if 0 <= tid < len(self.types) else 0
            if skip_special and ty in (CONTROL, UNKNOWN):
                continue
            piece = self.decode_one(tid)
            if first and self.add_space_prefix and piece[:1] == b" ":
                piece = piece[1:]
            if ty not in (CONTROL, UNKNOWN):
                first = False
            out += piece
        return out
