"""Public function signatures of a Rust source file, for comparing the safe
wrapper (crates/ramvamp-attn/src/lib.rs) with the reference's interface.

`signatures(text)` returns one entry per `pub fn`: its name, the `impl`
block it belongs to (None for a free function), its parameters as
(name, type) pairs in order (`self` forms as ("self", "&self") ...), and its
return type, all with whitespace normalised. Generic bounds and `where`
clauses are not used by either file and are not handled.
"""
from __future__ import annotations

import re


def _norm(t: str) -> str:
    t = " ".join(t.split())
    t = re.sub(r"\s*([<>(),\[\]&;:])\s*", r"\1", t)
    return t.replace("&mut", "&mut ").replace("&mut  ", "&mut ").strip()


def _split_top(s: str) -> list[str]:
    out, depth, cur = [], 0, []
    for ch in s:
        if ch in "<([":
            depth += 1
        elif ch in ">)]":
            depth -= 1
        if ch == "," and depth == 0:
            out.append("".join(cur))
            cur = []
        else:
            cur.append(ch)
    if "".join(cur).strip():
        out.append("".join(cur))
    return [x.strip() for x in out if x.strip()]


def _blocks(text: str):
    """(owner, start, end) of every top-level `impl Name {` block."""
    res = []
    for m in re.finditer(r"^impl(?:<[^>]*>)?\s+(\w+)\s*\{", text, flags=re.M):
        depth, i = 0, m.end() - 1
        while i < len(text):
            if text[i] == "{":
                depth += 1
            elif text[i] == "}":
                depth -= 1
                if depth == 0:
                    break
            i += 1
        res.append((m.group(1), m.start(), i))
    return res


def _strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", lambda m: " " * len(m.group(0)), text, flags=re.S)
    return re.sub(r"//[^\n]*", lambda m: " " * len(m.group(0)), text)


def signatures(text: str, lo: int = 0, hi: int | None = None):
    """Signatures of the `pub fn`s starting on lines lo..hi (1-based,
    inclusive; all when hi is None)."""
    text = _strip_comments(text)
    blocks = _blocks(text)
    starts = [0]
    for ln in text.splitlines(keepends=True):
        starts.append(starts[-1] + len(ln))
    out = []
    for m in re.finditer(r"\bpub fn (\w+)\s*(<[^>]*>)?\s*\(", text):
        line = text.count("\n", 0, m.start()) + 1
        if line < lo or (hi is not None and line > hi):
            continue
        depth, i = 1, m.end()
        while depth:
            if text[i] == "(":
                depth += 1
            elif text[i] == ")":
                depth -= 1
            i += 1
        params_s = text[m.end():i - 1]
        j = text.index("{", i)
        tail = text[i:j].strip()
        ret = _norm(tail[2:]) if tail.startswith("->") else "()"
        params = []
        for p in _split_top(params_s):
            flat = p.replace(" ", "")
            if flat in ("&self", "&mutself", "self", "mutself"):
                params.append(("self", {"&self": "&self", "&mutself": "&mut self"}.get(flat, "self")))
            else:
                name, ty = p.split(":", 1)
                params.append((name.strip(), _norm(ty)))
        owner = next((o for o, a, b in blocks if a < m.start() < b), None)
        out.append({"name": m.group(1), "owner": owner, "params": params, "ret": ret, "line": line})
    return out


def enum_variants(text: str, name: str):
    """{variant: [field names]} of `pub enum name { ... }` (struct-like
    variants list their fields; tuple variants list none)."""
    text = _strip_comments(text)
    m = re.search(r"pub enum " + name + r"\s*\{", text)
    depth, i = 1, m.end()
    while depth:
        depth += {"{": 1, "}": -1}.get(text[i], 0)
        i += 1
    body = re.sub(r"#\[[^\]]*\]", " ", text[m.end():i - 1])
    out = {}
    for v in re.finditer(r"\b([A-Z]\w*)\s*(\{[^}]*\}|\([^)]*\))?\s*,?", body):
        if v.group(2) and v.group(2).startswith("{"):
            out[v.group(1)] = re.findall(r"(\w+)\s*:", v.group(2))
        else:
            out[v.group(1)] = []
    return out
