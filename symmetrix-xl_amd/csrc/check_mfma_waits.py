#!/usr/bin/env python3
"""Checks this library's gfx950 assembly for MFMA results read too early.

An instruction that reads a register written by v_mfma_f32_16x16x4_f32 (8
passes) must issue at least ten wait states after it, on every path; the
hardware does not interlock.  The compiler inserts the waits, but in kernels
whose MFMA chains sat in runtime-conditional blocks it padded only the
fall-through path into a join, and a read on the taken branch came one
instruction after its MFMA (a stale accumulator element, silently wrong).
This walks each kernel's control-flow graph backwards from every instruction
that reads a register (VALU sources, memory addresses and data) and reports
the reads with fewer than MIN wait states since an MFMA that writes the
register, over any path; an s_nop N counts N + 1, other instructions one.

    python3 check_mfma_waits.py file.s [--min 10]      (exit 1 on findings)

The assembly comes from `make check-waits` (hipcc --cuda-device-only -S of
the sources that issue MFMAs).
"""

import argparse
import re
import sys
from collections import defaultdict

_BRANCH = re.compile(r"s_(?:c?branch\w*)\s+(\.LBB\w+)")
_RANGE = re.compile(r"([av])\[(\d+):(\d+)\]$")
_SINGLE = re.compile(r"([av])(\d+)$")


def _regs(token):
    token = token.strip()
    m = _RANGE.match(token)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = _SINGLE.match(token)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _cost(ins):
    m = re.match(r"s_nop\s+(\d+)", ins)
    return int(m.group(1)) + 1 if m else 1


def split_kernels(lines):
    """(name, body lines) per function of an assembly listing."""
    out, cur = [], None
    for ln in lines:
        m = re.match(r"^(_Z\S+|[A-Za-z_]\w*):(\s|$)", ln)
        if m and not ln.startswith("."):
            cur = (m.group(1), [])
            out.append(cur)
        elif cur is not None:
            cur[1].append(ln)
    return out


def _blocks(body):
    blocks, labels = [], {}
    cur = {"label": "<entry>", "ins": []}
    for ln in body:
        m = re.match(r"^(\.LBB\w+):", ln)
        if m:
            blocks.append(cur)
            cur = {"label": m.group(1), "ins": []}
            labels[m.group(1)] = len(blocks)
            continue
        text = ln.split(";")[0].strip()
        if not text or text.startswith("."):
            continue
        cur["ins"].append(text)
        if text.startswith("s_endpgm"):
            break
        if text.startswith("s_cbranch") or text.startswith("s_branch"):
            # a branch ends its block: the taken edge leaves from here, the next instruction falls through
            blocks.append(cur)
            cur = {"label": "<after %s>" % text.split()[0], "ins": []}
    blocks.append(cur)
    preds = defaultdict(set)
    for i, b in enumerate(blocks):
        for ins in b["ins"]:
            m = _BRANCH.match(ins)
            if m and m.group(1) in labels:
                preds[labels[m.group(1)]].add(i)
        last = b["ins"][-1] if b["ins"] else ""
        if not (last.startswith("s_branch") or last.startswith("s_endpgm")) and i + 1 < len(blocks):
            preds[i + 1].add(i)
    return blocks, preds


def findings(body, minimum):
    """(block label, instruction, register, wait states) for each early read."""
    blocks, preds = _blocks(body)

    def since_mfma(bi, idx, reg, budget, seen):
        ins = blocks[bi]["ins"]
        d = 0
        for k in range(idx - 1, -1, -1):
            t = ins[k]
            if t.startswith("v_mfma") and reg in _regs(t.split(None, 1)[1].split(",")[0]):
                return d
            d += _cost(t)
            if d >= budget:
                return budget
        best = budget
        for p in preds[bi]:
            if (p, reg) not in seen:
                best = min(best, d + since_mfma(p, len(blocks[p]["ins"]), reg, budget - d, seen | {(p, reg)}))
        return best

    out = []
    for bi, b in enumerate(blocks):
        for k, t in enumerate(b["ins"]):
            if t.startswith("v_mfma") or t.startswith("s_") or " " not in t:
                continue
            ops = t.split(None, 1)[1].split(",")
            for op in (ops[1:] if t.startswith("v_") else ops):
                for reg in _regs(op):
                    d = since_mfma(bi, k, reg, minimum, frozenset())
                    if d < minimum:
                        out.append((b["label"], t, "%s%d" % reg, d))
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("asm", nargs="+")
    ap.add_argument("--min", type=int, default=10)
    args = ap.parse_args(argv)
    bad = 0
    for path in args.asm:
        with open(path) as f:
            kernels = split_kernels(f.read().split("\n"))
        for name, body in kernels:
            for label, ins, reg, d in findings(body, args.min):
                bad += 1
                print("%s: %s: %s: %s read %d wait states after its MFMA" % (path, name, label, ins, d))
        print("%s: %d functions checked" % (path, len(kernels)))
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main())
