"""Mechanical rewrite of a libsbsa .hip source into host C++ for the CPU emulation
(tests/emu/include/hip/hip_runtime.h).  Test infrastructure only.

The kernel code itself is kept as written.  What changes:
- address-space qualifiers are dropped (LDS and constant pointers are plain host
  pointers; the emulation maps 32-bit LDS addresses back);
- ``extern __shared__`` dynamic LDS becomes the emulator's LDS arena;
- each inline-assembly statement is replaced by the emulation of what it does,
  chosen by its template (loads straight into LDS, written MFMAs, accumulation
  register reads and zeroing, wait states and register laundering, which do
  nothing on the host).  An assembly statement that matches no known template
  stops the rewrite.
"""
from __future__ import annotations

import re
import sys
from pathlib import Path


def _balanced(text: str, start: int) -> int:
    """Index just past the parenthesis that closes the one at text[start]."""
    depth, i, in_str = 0, start, False
    while i < len(text):
        ch = text[i]
        if in_str:
            if ch == "\\":
                i += 2
                continue
            if ch == '"':
                in_str = False
        elif ch == '"':
            in_str = True
        elif ch == "(":
            depth += 1
        elif ch == ")":
            depth -= 1
            if depth == 0:
                return i + 1
        i += 1
    raise ValueError("unbalanced asm statement")


def _split_colons(body: str) -> list[str]:
    parts, depth, cur, in_str, i = [], 0, [], False, 0
    while i < len(body):
        ch = body[i]
        if in_str:
            cur.append(ch)
            if ch == "\\":
                cur.append(body[i + 1])
                i += 2
                continue
            if ch == '"':
                in_str = False
        elif ch == '"':
            in_str = True
            cur.append(ch)
        elif ch in "([":
            depth += 1
            cur.append(ch)
        elif ch in ")]":
            depth -= 1
            cur.append(ch)
        elif ch == ":" and depth == 0:
            parts.append("".join(cur))
            cur = []
        else:
            cur.append(ch)
        i += 1
    parts.append("".join(cur))
    return parts


def _operands(spec: str) -> list[tuple[str, str]]:
    """'"=v"(x), "v"(y)' -> [('=v', 'x'), ('v', 'y')]"""
    out = []
    for m in re.finditer(r'"([^"]*)"\s*\(', spec):
        end = _balanced(spec, m.end() - 1)
        out.append((m.group(1), spec[m.end():end - 1].strip()))
    return out


def _template(part: str) -> str:
    return "".join(re.findall(r'"((?:[^"\\]|\\.)*)"', part)).replace("\\n", "\n").replace("\\t", "\t")


def _rewrite_asm(stmt_body: str) -> str:
    parts = _split_colons(stmt_body)
    tpl = _template(parts[0]).strip()
    outs = _operands(parts[1]) if len(parts) > 1 else []
    ins = _operands(parts[2]) if len(parts) > 2 else []
    words = tpl.split()
    if tpl == "":
        return "(void)0"                                   # register laundering
    if all(w.startswith("s_nop") or w.isdigit() for w in words):
        return "(void)0"                                   # wait states
    if "buffer_load_dwordx4" in tpl and " lds" in tpl:
        (_, lds), (_, voff), (_, rsrc) = ins
        return (f"{{ uint32_t r_[4] = {{({rsrc}).x, ({rsrc}).y, ({rsrc}).z, ({rsrc}).w}}; "
                f"emu::buffer_load_lds(r_, {lds}, {voff}, 16); }}")
    if "buffer_load_dword " in tpl and " lds" in tpl:
        (_, lds), (_, voff), (_, rsrc) = ins
        return (f"{{ uint32_t r_[4] = {{({rsrc}).x, ({rsrc}).y, ({rsrc}).z, ({rsrc}).w}}; "
                f"emu::buffer_load_lds(r_, {lds}, {voff}, 4); }}")
    m = re.fullmatch(r"(?:s_nop \d+\s+)?v_mfma_f32_32x32x16_bf16 %0, %(\d), %(\d), (0|%0)", tpl)
    if m:
        (_, d), = outs
        a = ins[int(m.group(1)) - 1][1] if m.group(1) != "0" else d
        b = ins[int(m.group(2)) - 1][1] if m.group(2) != "0" else d
        acc = d if m.group(3) == "%0" else f"std::remove_reference_t<decltype({d})>{{}}"
        return f"{d} = emu::mfma32x32x16({a}, {b}, {acc})"
    if re.fullmatch(r"v_accvgpr_read_b32 %0, %1", tpl):
        (_, v), = outs
        (_, a), = ins
        return f"{v} = {a}"
    raise ValueError(f"no emulation for asm template {tpl!r}")


def transform(src: str) -> str:
    src = re.sub(r"__attribute__\(\(address_space\(\d\)\)\)\s*", "", src)
    src = re.sub(r"extern\s+__shared__\s+(?:__attribute__\(\(aligned\(\d+\)\)\)\s*)?([\w ]+?)\s+(\w+)\s*\[\s*\]\s*;",
                 r"\1* \2 = (\1*)emu::dyn_lds();", src)
    # static LDS: each declaration registers the array, so that the emulation
    # fills it with stale bytes when a block starts (as LDS holds on the GPU)
    src = re.sub(r"(?m)^(\s*)__shared__\s+([^;()]*?(?:__attribute__\(\(aligned\(\d+\)\)\)\s*)?[^;()]*?)\b(\w+)\s*((?:\[[^\];]*\])+)\s*;",
                 r"\1static \2\3\4; emu::shared_var(\3, sizeof(\3));", src)
    out, i = [], 0
    for m in re.finditer(r"\basm\s+volatile\s*\(|\basm\s*\(", src):
        if m.start() < i:
            continue
        end = _balanced(src, m.end() - 1)
        out.append(src[i:m.start()])
        out.append(_rewrite_asm(src[m.end():end - 1]))
        i = end
    out.append(src[i:])
    text = "".join(out)
    if re.search(r"\basm\s+volatile\s*\(|\basm\s*\(", text):
        raise ValueError("assembly left after the rewrite")
    return text


if __name__ == "__main__":
    Path(sys.argv[2]).write_text(transform(Path(sys.argv[1]).read_text()))
