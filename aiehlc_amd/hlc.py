"""Source-to-source front end: aiehlc host sources retargeted to gfx950.

aiehlc (src/llvm/aiehlc.cc:469-607, with the AST pass at :150-330) takes a
host program that declares AI Engine kernels inline and produces host code
for the ARM core:
  - every `__global__` / `__kernel__` function definition is cut out of the
    host source (its text becomes an AIE kernel source);
  - a `__global__` kernel is loaded by XAie_LoadElfMem, whose last argument
    is rewritten to the embedded ELF `_binary_kernel_<name>_start`;
  - a `__kernel__` name gets a template
        template <int Col, int Row, int colstart, int rowstart, int M, int N, int K,
                  typename... Args> inline void NAME(Args&&... args)
    prepended, which today does nothing.

This module performs the same rewrite for MI355X:
  - the definitions are cut out the same way (the line count is kept, so
    compiler messages still point at the original lines);
  - XAie_LoadElfMem's last argument becomes the gfx950 kernel descriptor
    (`&miaie_xaie_mm` ...), which the aie-rt-shaped facade
    (include/miaie_xaie.h) runs on its tile memories;
  - the `__kernel__` template forwards to miaie_hlc::launch
    (include/miaie_hlc.hpp): device pointers go to the miaie launch
    templates, DDR addresses to the tiles the template arguments name;
  - `#include "xaiengine.h"` becomes `#include "miaie_xaie.h"`.

Which gfx950 kernel a definition maps to is decided by keyword, name and
parameter types (table below), or given explicitly with --map NAME=TARGET.
A kernel with no counterpart is an error: it is reported, never dropped.

    python -m aiehlc_amd.hlc input.cc -o host.cc [--kernel-list FILE] [--map NAME=TARGET]
"""
from __future__ import annotations

import argparse
import dataclasses
import re
import sys

# `__global__` targets: XAie_MiaieKernel descriptors of the facade.
GLOBAL_TARGETS = {"mm": "miaie_xaie_mm", "perf": "miaie_xaie_perf", "k1": "miaie_xaie_k1", "k2": "miaie_xaie_k2",
                  "mm3_u64": "miaie_xaie_mm3_u64", "perf_u8": "miaie_xaie_perf_u8"}
# `__kernel__` targets: miaie_hlc::Kernel values.
KERNEL_TARGETS = {"perf_u8": "perf_u8", "mm": "mm", "perf": "perf", "gemm_i8": "gemm_i8", "gemm_bf16": "gemm_bf16"}

BSP_HEADERS = ("xil_printf.h", "xil_cache.h", "xtime_l.h", "xiltimer.h", "xil_io.h")


class HlcError(Exception):
    pass


@dataclasses.dataclass
class Param:
    text: str
    type: str            # declared type with annotations removed, e.g. "input_window_int32 *"
    name: str
    mem_address: int = 0
    size_hint: int = 0


@dataclasses.dataclass
class KernelDef:
    keyword: str         # "__global__" or "__kernel__"
    name: str
    params: list
    start: int           # span of the definition in the source
    end: int
    target: str = ""
    ping: list = dataclasses.field(default_factory=list)


# ------------------------------------------------------------------ lexing
def code_mask(src: str) -> list[bool]:
    """True for characters that are code: not inside a comment or a string
    or character literal."""
    mask = [True] * len(src)
    i, n = 0, len(src)
    while i < n:
        c = src[i]
        if src.startswith("//", i):
            j = src.find("\n", i)
            j = n if j < 0 else j
            for k in range(i, j):
                mask[k] = False
            i = j
        elif src.startswith("/*", i):
            j = src.find("*/", i + 2)
            j = n if j < 0 else j + 2
            for k in range(i, j):
                mask[k] = False
            i = j
        elif c in "\"'":
            j = i + 1
            while j < n and src[j] != c:
                j += 2 if src[j] == "\\" else 1
            j = min(j + 1, n)
            for k in range(i, j):
                mask[k] = False
            i = j
        else:
            i += 1
    return mask


def _match(src: str, mask: list[bool], i: int, open_c: str, close_c: str) -> int:
    """Index just past the bracket that closes the one at src[i]."""
    depth = 0
    for j in range(i, len(src)):
        if not mask[j]:
            continue
        if src[j] == open_c:
            depth += 1
        elif src[j] == close_c:
            depth -= 1
            if depth == 0:
                return j + 1
    raise HlcError(f"unbalanced '{open_c}' at offset {i}")


def _split_top(text: str, mask_off: int, mask: list[bool], sep: str = ",") -> list[str]:
    parts, depth, cur = [], 0, []
    for k, ch in enumerate(text):
        code = mask[mask_off + k]
        if code and ch in "([{":
            depth += 1
        elif code and ch in ")]}":
            depth -= 1
        if code and ch == sep and depth == 0:
            parts.append("".join(cur))
            cur = []
        else:
            cur.append(ch)
    parts.append("".join(cur))
    return [p for p in (x.strip() for x in parts) if p]


_ANNOT = re.compile(r'annotate\s*\(\s*"(mem_address|size_hint)\s*:\s*([0-9a-fA-Fx]+)"\s*\)')
_ATTR = re.compile(r"__attribute__\s*\(\(")


def _strip_attributes(text: str) -> str:
    out = text
    while True:
        m = _ATTR.search(out)
        if not m:
            return out
        depth, j = 0, m.start() + len("__attribute__")
        while j < len(out):
            if out[j] == "(":
                depth += 1
            elif out[j] == ")":
                depth -= 1
                if depth == 0:
                    break
            j += 1
        out = out[:m.start()] + out[j + 1:]


def _parse_param(text: str) -> Param:
    p = Param(text=text, type="", name="")
    for key, val in _ANNOT.findall(text):
        setattr(p, key, int(val, 0))
    bare = " ".join(_strip_attributes(text).split())
    m = re.match(r"^(.*?)([A-Za-z_]\w*)\s*$", bare)
    if not m:
        raise HlcError(f"cannot read parameter '{text}'")
    p.type, p.name = m.group(1).strip(), m.group(2)
    return p


def find_kernels(src: str, mask: list[bool] | None = None) -> list[KernelDef]:
    """Every `__global__` / `__kernel__` function definition (or declaration)
    outside comments and strings, in source order."""
    mask = code_mask(src) if mask is None else mask
    out = []
    for m in re.finditer(r"\b(__global__|__kernel__)\b", src):
        if not mask[m.start()]:
            continue
        paren = src.find("(", m.end())
        while paren >= 0 and not mask[paren]:
            paren = src.find("(", paren + 1)
        if paren < 0:
            raise HlcError(f"{m.group(1)} at offset {m.start()} has no parameter list")
        head = src[m.end():paren]
        nm = re.search(r"([A-Za-z_]\w*)\s*$", head)
        if not nm:
            raise HlcError(f"no kernel name before '(' at offset {paren}")
        close = _match(src, mask, paren, "(", ")")
        params = [_parse_param(t) for t in _split_top(src[paren + 1:close - 1], paren + 1, mask)]
        if len(params) == 1 and params[0].type in ("", "void") and params[0].name == "void":
            params = []
        j = close
        while j < len(src) and (src[j].isspace() or not mask[j]):
            j += 1
        if j < len(src) and src[j] == "{":
            end = _match(src, mask, j, "{", "}")
        elif j < len(src) and src[j] == ";":
            end = j + 1
        else:
            raise HlcError(f"{m.group(1)} {nm.group(1)}: expected a body or ';' after the parameters")
        out.append(KernelDef(m.group(1), nm.group(1), params, m.start(), end))
    return out


# ------------------------------------------------------------------ mapping
def window_layout(params: list[Param]) -> list[int]:
    """Ping addresses by the reference compiler's placement rule
    (src/mlir/mlirfront/AieFrontEnd.cc:297-394): the first window starts at
    0x1000 unless annotated; each reserves 4*size_hint words (512 by
    default) for ping and again for pong; an annotation moves a window."""
    addr, ping = 0x1000, []
    for p in params:
        words = 4 * (p.size_hint or 512)
        if p.mem_address:
            addr = p.mem_address
        ping.append(addr)
        addr += 2 * words * 4
    return ping


def _default_target(k: KernelDef) -> str:
    types = [p.type.replace(" ", "") for p in k.params]
    windows = all("window" in t for t in types) and len(types) == 2
    if k.keyword == "__global__":
        if k.name in ("mm", "perf") and windows:
            return GLOBAL_TARGETS[k.name]
        if k.name == "mm" and types == ["uint64_t*", "uint64_t*"]:
            return GLOBAL_TARGETS["mm3_u64"]
        if k.name in ("k1", "k2") and types == ["int*", "int*"]:
            return GLOBAL_TARGETS[k.name]
        return ""
    # __kernel__: example/nokernelload's `perf` is the uint8 MAC probe
    if k.name == "perf" and windows:
        return KERNEL_TARGETS["perf_u8"]
    if k.name in ("mm", "gemm_i8", "gemm_bf16"):
        return KERNEL_TARGETS[k.name]
    return ""


def resolve(kernels: list[KernelDef], overrides: dict[str, str]) -> None:
    missing = []
    for k in kernels:
        if k.name in overrides:
            t = overrides[k.name]
            table = GLOBAL_TARGETS if k.keyword == "__global__" else KERNEL_TARGETS
            if t not in table:
                raise HlcError(f"--map {k.name}={t}: unknown {k.keyword} target (choose from {', '.join(table)})")
            k.target = table[t]
        else:
            k.target = _default_target(k)
        if not k.target:
            missing.append(f"{k.keyword} {k.name}({', '.join(p.type for p in k.params)})")
        k.ping = window_layout(k.params)
    if missing:
        raise HlcError("no gfx950 counterpart for: " + "; ".join(missing) +
                       " (name one with --map NAME=TARGET)")


# ------------------------------------------------------------------ rewrite
def _blank(text: str, note: str) -> str:
    """A comment standing for a removed definition, with its line count."""
    return f"/* {note} */" + "\n" * text.count("\n")


def _forwarder(name: str, target: str) -> str:
    return ("template <int Col, int Row, int colstart, int rowstart, int M, int N, int K, typename... Args>\n"
            f"inline void {name}(Args&&... args) {{\n"
            f"  miaie_hlc::launch<miaie_hlc::Kernel::{target}, Col, Row, colstart, rowstart, M, N, K>("
            "std::forward<Args>(args)...);\n}\n")


def rewrite(src: str, overrides: dict[str, str] | None = None,
            filename: str = "") -> tuple[str, list[KernelDef], list[str]]:
    """Return (host source, kernels, warnings).  With `filename`, compiler
    messages on the output point at that file's lines."""
    mask = code_mask(src)
    kernels = find_kernels(src, mask)
    resolve(kernels, overrides or {})
    globals_ = {k.name: k for k in kernels if k.keyword == "__global__"}
    edits = []  # (start, end, replacement)
    for k in kernels:
        edits.append((k.start, k.end, _blank(src[k.start:k.end], f"{k.keyword} {k.name}: gfx950 kernel {k.target}")))
    # XAie_LoadElfMem(dev, loc, <kernel>): the last argument names a __global__ kernel
    for m in re.finditer(r"\bXAie_LoadElfMem\s*\(", src):
        if not mask[m.start()] or any(s <= m.start() < e for s, e, _ in edits):
            continue
        open_i = m.end() - 1
        close = _match(src, mask, open_i, "(", ")")
        args = _split_top(src[open_i + 1:close - 1], open_i + 1, mask)
        if len(args) != 3:
            raise HlcError(f"XAie_LoadElfMem with {len(args)} arguments at offset {m.start()}")
        ident = re.findall(r"[A-Za-z_]\w*", args[2])
        kname = ident[-1] if ident else ""
        if kname not in globals_:
            raise HlcError(f"XAie_LoadElfMem loads '{args[2]}', which is not a __global__ kernel of this file")
        new = f"XAie_LoadElfMem({args[0]}, {args[1]}, (const unsigned char *)&{globals_[kname].target})"
        edits.append((m.start(), close, new + "\n" * src[m.start():close].count("\n")))  # keep the line count
    warnings = []
    for m in re.finditer(r'#\s*include\s*[<"]([^>"]+)[>"]', src):
        if not mask[m.start()] and not mask[m.end() - 1]:
            continue
        header = m.group(1)
        if header == "xaiengine.h":
            edits.append((m.start(), m.end(), '#include "miaie_xaie.h"'))
        elif header in BSP_HEADERS:
            warnings.append(f"#include \"{header}\": a Xilinx BSP header; supply a host replacement")
    out, last = [], 0
    for s, e, r in sorted(edits):
        if s < last:
            raise HlcError(f"overlapping rewrites at offset {s}")
        out.append(src[last:s])
        out.append(r)
        last = e
    out.append(src[last:])
    body = "".join(out)
    knames = [k for k in kernels if k.keyword == "__kernel__"]
    prefix = ("// Rewritten for gfx950 by aiehlc_amd/hlc.py: __global__ / __kernel__ definitions run as\n"
              "// miaie kernels (kernel list below).\n")
    for k in kernels:
        prefix += f"//   {k.keyword} {k.name} -> {k.target} (windows at {', '.join(hex(p) for p in k.ping)})\n"
    if knames:
        prefix += "#include <utility>\n#include \"miaie_hlc.hpp\"\n"
        for k in knames:
            prefix += _forwarder(k.name, k.target)
    line = f'#line 1 "{filename}"\n' if filename else "#line 1\n"
    return prefix + line + body, kernels, warnings


def kernel_list(kernels: list[KernelDef]) -> str:
    """One line per kernel, like the reference's `kernel_list` output
    (aiehlc.cc:63-82), with the gfx950 target and window addresses."""
    return "".join(f"{k.name} {k.keyword} {k.target} {' '.join(hex(p) for p in k.ping)}\n" for k in kernels)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("input")
    ap.add_argument("-o", "--output", required=True)
    ap.add_argument("--kernel-list")
    ap.add_argument("--map", action="append", default=[], metavar="NAME=TARGET")
    args = ap.parse_args(argv)
    overrides = {}
    for item in args.map:
        name, _, target = item.partition("=")
        if not name or not target:
            ap.error(f"--map {item}: expected NAME=TARGET")
        overrides[name] = target
    try:
        out, kernels, warnings = rewrite(open(args.input).read(), overrides, filename=args.input)
    except HlcError as e:
        print(f"hlc: {args.input}: {e}", file=sys.stderr)
        return 1
    for w in warnings:
        print(f"hlc: {args.input}: warning: {w}", file=sys.stderr)
    with open(args.output, "w") as f:
        f.write(out)
    if args.kernel_list:
        with open(args.kernel_list, "w") as f:
            f.write(kernel_list(kernels))
    return 0


if __name__ == "__main__":
    sys.exit(main())
