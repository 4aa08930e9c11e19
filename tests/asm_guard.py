"""Static checks of the HIP sources and of the compiler's resource-usage remarks
that keep the kernels' inline-asm memory instructions within the rules they
were written to (CPU only; used by tests/test_asm_guard.py).

1. Every inline-asm statement whose template issues a vector memory
   instruction opens with ``KF_VMEM_ASM_NOPS`` (``s_nop 4``): the compiler does
   not insert the wait states the ISA requires in front of an asm statement, so
   an SGPR written by a VALU instruction (a ``v_readlane`` reload) or m0 written
   just before could be read stale as the address base.
2. No inline-asm memory instruction has register outputs: an asm load into
   registers is invisible to the compiler's wait counting, and when the
   destination lives in an array the compiler may place in scratch memory, the
   load lands there asynchronously.  The kernels' asm loads go global -> LDS.
3. A kernel that reaches an asm direct-to-LDS load (directly or through the
   device functions it calls) uses no scratch memory: its registers all live in
   the register file, so no spill or reload can sit next to the asm.
"""

from __future__ import annotations

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "kempnerforge_amd", "csrc")
OBJ = os.path.join(ROOT, "kempnerforge_amd", "lib", "obj")

NOPS_MACRO = "KF_VMEM_ASM_NOPS"
_VMEM = re.compile(r"\b(global|buffer|flat|scratch)_(load|store|atomic)\w*")


def sources() -> dict[str, str]:
    """name -> text of every HIP source and header of the library."""
    out = {}
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".hip", ".h")):
            with open(os.path.join(CSRC, name)) as f:
                out[name] = f.read()
    return out


def strip_comments(text: str) -> str:
    """Removes // and /* */ comments, keeping string literals and line count."""
    out, i, n = [], 0, len(text)
    while i < n:
        c = text[i]
        if c == '"':
            j = i + 1
            while j < n and text[j] != '"':
                j += 2 if text[j] == "\\" else 1
            out.append(text[i:j + 1])
            i = j + 1
        elif text.startswith("//", i):
            j = text.find("\n", i)
            i = n if j < 0 else j
        elif text.startswith("/*", i):
            j = text.find("*/", i + 2)
            seg = text[i:(n if j < 0 else j + 2)]
            out.append("\n" * seg.count("\n"))
            i = n if j < 0 else j + 2
        else:
            out.append(c)
            i += 1
    return "".join(out)


def _match(text: str, i: int, open_c: str, close_c: str) -> int:
    """Index just past the bracket closing the one at text[i] (strings skipped)."""
    depth, n = 0, len(text)
    while i < n:
        c = text[i]
        if c == '"':
            i += 1
            while i < n and text[i] != '"':
                i += 2 if text[i] == "\\" else 1
        elif c == open_c:
            depth += 1
        elif c == close_c:
            depth -= 1
            if depth == 0:
                return i + 1
        i += 1
    raise ValueError("unbalanced brackets")


def _split_top(s: str, sep: str) -> list[str]:
    """Splits s at top-level occurrences of sep (outside brackets and strings)."""
    parts, depth, cur, i = [], 0, [], 0
    while i < len(s):
        c = s[i]
        if c == '"':
            j = i + 1
            while j < len(s) and s[j] != '"':
                j += 2 if s[j] == "\\" else 1
            cur.append(s[i:j + 1])
            i = j + 1
            continue
        if c in "([{":
            depth += 1
        elif c in ")]}":
            depth -= 1
        if c == sep and depth == 0:
            parts.append("".join(cur))
            cur = []
        else:
            cur.append(c)
        i += 1
    parts.append("".join(cur))
    return parts


def asm_statements(text: str) -> list[tuple[int, str, str]]:
    """(line, template, outputs) of every inline-asm statement: the template is
    the part before the first top-level ':' (macros and literals as written),
    outputs the operand list after it."""
    code = strip_comments(text)
    out = []
    for m in re.finditer(r"\b(?:asm|__asm__)\s*(?:volatile|__volatile__)?\s*\(", code):
        start = m.end() - 1
        end = _match(code, start, "(", ")")
        parts = _split_top(code[start + 1:end - 1], ":")
        line = code.count("\n", 0, m.start()) + 1
        out.append((line, parts[0].strip(), parts[1].strip() if len(parts) > 1 else ""))
    return out


def check_asm(text: str, name: str = "<source>") -> list[str]:
    """Violations of rules 1 and 2 in one source text."""
    bad = []
    for line, template, outputs in asm_statements(text):
        literal = "".join(re.findall(r'"((?:[^"\\]|\\.)*)"', template))
        if not _VMEM.search(literal):
            continue
        if not template.startswith(NOPS_MACRO):
            bad.append(f"{name}:{line}: asm memory instruction without {NOPS_MACRO} in front")
        if outputs:
            bad.append(f"{name}:{line}: asm memory instruction with register outputs ({outputs})")
    return bad


def _definitions(code: str) -> dict[str, str]:
    """name -> body text of every function defined with __global__ or __device__
    (bodies of overloads and template instances of one name concatenated)."""
    defs: dict[str, str] = {}
    for m in re.finditer(r"\b(__global__|__device__)\b", code):
        # the declarator: the first identifier followed by '(' after the
        # qualifiers, return type and any __launch_bounds__(...) / attributes
        j = m.end()
        while True:
            nm = re.compile(r"\s*([A-Za-z_]\w*)\s*(\(|<|::|\*|&|\s)").match(code, j)
            if nm is None:
                break
            ident, nxt = nm.group(1), nm.group(2)
            if nxt == "(" and ident in ("__launch_bounds__", "__attribute__", "__align__",
                                        "alignas"):
                j = _match(code, code.index("(", nm.start(1)), "(", ")")
                continue
            if nxt == "(":
                break
            if nxt == "<":  # a template type such as f32x16 or std::array<...>
                j = _match(code, code.index("<", nm.start(1)), "<", ">")
                continue
            j = nm.end(1)
        if nm is None or nm.group(2) != "(":
            continue
        name = nm.group(1)
        params_end = _match(code, code.index("(", nm.start(1)), "(", ")")
        rest = code[params_end:params_end + 400]
        semi, brace = rest.find(";"), rest.find("{")
        if brace < 0 or (0 <= semi < brace):
            continue  # a declaration, or a __device__ variable
        body_start = params_end + brace
        body = code[body_start:_match(code, body_start, "{", "}")]
        defs[name] = defs.get(name, "") + body
    return defs


def dma_functions(texts: dict[str, str]) -> set[str]:
    """Names of the __global__ / __device__ functions that reach an inline-asm
    vector memory instruction, directly or through other such functions."""
    code = "\n".join(strip_comments(t) for t in texts.values())
    defs = _definitions(code)
    reach = {n for n, body in defs.items()
             if any(_VMEM.search("".join(re.findall(r'"((?:[^"\\]|\\.)*)"', tpl)))
                    for _, tpl, _ in asm_statements(body))}
    changed = True
    while changed:
        changed = False
        for n, body in defs.items():
            if n in reach:
                continue
            if any(re.search(r"\b%s\b" % re.escape(r), body) for r in reach):
                reach.add(n)
                changed = True
    return reach


def kernels(texts: dict[str, str]) -> set[str]:
    code = "\n".join(strip_comments(t) for t in texts.values())
    return {n for n in _definitions(code)
            if re.search(r"__global__[^;{(]*(?:\([^)]*\)[^;{(]*)?\b%s\s*\(" % re.escape(n), code)}


def parse_remarks(text: str) -> dict[str, dict[str, int]]:
    """mangled kernel name -> {'VGPRs', 'AGPRs', 'ScratchSize', 'VGPRs Spill', ...}
    from the output of -Rpass-analysis=kernel-resource-usage."""
    out: dict[str, dict[str, int]] = {}
    cur = None
    for line in text.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            out[cur] = {}
            continue
        m = re.search(r"remark:\s+([A-Za-z ]+?)(?: \[[^\]]*\])?: (\d+)", line)
        if m and cur is not None:
            out[cur][m.group(1)] = int(m.group(2))
    return out


def source_name(mangled: str, names: set[str]) -> str | None:
    """The source-level name (one of ``names``) a mangled kernel symbol carries."""
    hits = [n for n in names if f"{len(n)}{n}" in mangled]
    return max(hits, key=len) if hits else None


def check_scratch(remarks: dict[str, dict[str, int]], dma: set[str]) -> list[str]:
    """Violations of rule 3: kernels reaching an asm load with scratch in use."""
    bad = []
    for mangled, info in sorted(remarks.items()):
        name = source_name(mangled, dma)
        if name is None:
            continue
        # (SGPR spills go to VGPR lanes, not scratch: their v_readlane reloads
        # are the hazard rule 1's wait states cover)
        if info.get("ScratchSize", 0) or info.get("VGPRs Spill", 0):
            bad.append(f"{name} ({mangled}): ScratchSize {info.get('ScratchSize')} bytes/lane, "
                       f"{info.get('VGPRs Spill')} VGPRs spilled")
    return bad
