"""The integration guide stays true to the C ABI: every l2c_ entry point it
names is declared in include/, and every call it writes out passes as many
arguments as the declaration takes."""
import os
import re

from conftest import ROOT

HEADERS = [os.path.join(ROOT, "include", h) for h in ("l2c.h", "l2c_harness.h")]
GUIDE = os.path.join(ROOT, "INTEGRATION.md")


def _split_args(text):
    """Top-level comma-separated arguments of a parenthesised list's body."""
    depth, cur, out = 0, [], []
    for ch in text:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append("".join(cur).strip())
            cur = []
        else:
            cur.append(ch)
    last = "".join(cur).strip()
    if last:
        out.append(last)
    return out


def _balanced(text, start):
    """The body of the parenthesised list opening at text[start] == '('."""
    depth = 0
    for i in range(start, len(text)):
        if text[i] == "(":
            depth += 1
        elif text[i] == ")":
            depth -= 1
            if depth == 0:
                return text[start + 1:i]
    raise ValueError("unbalanced parentheses")


def declarations():
    decls = {}
    for path in HEADERS:
        src = open(path).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        for m in re.finditer(r"\b(l2c_\w+)\s*\(", src):
            # a declaration: the name follows a return type and the list ends in ';'
            body = _balanced(src, m.end() - 1)
            tail = src[m.end() - 1 + len(body) + 2:].lstrip()
            if not tail.startswith(";"):
                continue
            params = _split_args(body)
            decls[m.group(1)] = 0 if params in ([], ["void"]) else len(params)
    return decls


def guide_calls():
    text = open(GUIDE).read()
    blocks = re.findall(r"```(?:cpp|c)\n(.*?)```", text, flags=re.S)
    calls = []
    for block in blocks:
        code = re.sub(r"//[^\n]*", "", block)
        for m in re.finditer(r"\b(l2c_\w+)\s*\(", code):
            calls.append((m.group(1), len(_split_args(_balanced(code, m.end() - 1)))))
    return text, calls


def test_headers_parse():
    decls = declarations()
    assert decls["l2c_rmsnorm"] == 7 and decls["l2c_softmax"] == 5 and decls["l2c_strerror"] == 1
    assert decls["l2c_matmul_q"] == 9 and decls["l2c_matmul_qs"] == 11


def test_every_named_entry_point_is_declared():
    decls = declarations()
    text, _ = guide_calls()
    named = set(re.findall(r"\b(l2c_[a-z0-9_]+)\s*\(", text))
    missing = sorted(n for n in named if n not in decls)
    assert not missing, missing


def test_guide_calls_match_declared_arity():
    decls = declarations()
    _, calls = guide_calls()
    assert len(calls) >= 15
    wrong = [(name, n, decls.get(name)) for name, n in calls if decls.get(name) != n]
    assert not wrong, wrong
