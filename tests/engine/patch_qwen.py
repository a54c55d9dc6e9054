#!/usr/bin/env python3
"""Print the reference engine (engines/qwen.c) with the om_hip hooks added.

Reads the reference file where it lies and writes the hooked translation unit
to stdout, which tests/engine/Makefile pipes straight into the compiler: no
copy of the reference source is written anywhere.  The hooks themselves live
in omh_qwen_hooks.h / omh_qwen_main.h (this build's code); what is inserted
here is only their #include lines and one macro line at each hook point,
found by the signature it follows, with #line directives so that compiler
messages keep pointing at the reference file's own lines.

Hook points (each must match exactly once, or the build fails):
  - deltanet_step (qwen.c:301): the GDN layer's GPU call;
  - attn_step (qwen.c:367): the attention layer's GPU call;
  - serve (qwen.c:566): the batched prompt step and the teacher-forced gate
    (omh_qwen_main.h) are included in front of it;
  - the reset branch of serve (qwen.c:576): device states reset too;
  - serve's prompt loop (qwen.c:588): the prompt as one batched step (unless
    OMH_BATCH_PROMPT=0);
  - main (qwen.c:616): the teacher-forced gate (--tf) and, in front of the
    prompt loop (qwen.c:637), the batched prompt step (OMH_BATCH_PROMPT=1).

usage: patch_qwen.py /path/to/engines/qwen.c > hooked.c
"""
import re
import sys

# (pattern of the anchor line, lines before it, lines after it)
HOOKS = [
    (r"static void deltanet_step\(Model \*m, Layer \*l, int li, const float \*x, float \*out\) \{",
     ['#include "omh_qwen_hooks.h"'], ["    OMH_GDN_HOOK(m, l, li, x, out);"]),
    (r"static void attn_step\(Model \*m, Layer \*l, int li, const float \*x, int pos, float \*out\) \{",
     [], ["    OMH_ATTN_HOOK(m, l, li, x, pos, out);"]),
    (r"static int serve\(const char \*snap\) \{",
     ['#include "omh_qwen_main.h"'], []),
    (r"\s*if \(reset\) \{",
     [], ["            OMH_RESET(&m);"]),
    (r"\s*for \(int i = 0; i < nids; i\+\+\) \{ free\(logit\); logit = step\(&m,\(int\)jids->kids\[i\]->num\); \}",
     ["        OMH_SERVE_PROMPT(&m, jids, nids, logit)"], []),
    (r"int main\(int argc, char \*\*argv\) \{",
     [], ["    OMH_MAIN_HOOK(argc, argv);"]),
    (r"\s*for \(int i = 0; i < np; i\+\+\) \{ free\(logit\); logit = step\(&m, prompt\[i\]\); \}",
     ["    OMH_PROMPT(&m, prompt, np, logit)"], []),
]


def main() -> int:
    if len(sys.argv) != 2:
        sys.exit(__doc__)
    path = sys.argv[1]
    with open(path) as f:
        lines = f.read().split("\n")
    found = {i: [] for i in range(len(HOOKS))}
    for n, line in enumerate(lines):
        for i, (pat, _, _) in enumerate(HOOKS):
            if re.fullmatch(pat, line.rstrip()):
                found[i].append(n)
    for i, hits in found.items():
        if len(hits) != 1:
            sys.exit(f"patch_qwen: hook point {HOOKS[i][0]!r} matched {len(hits)} lines of {path}")
    at = {hits[0]: i for i, hits in found.items()}
    out = [f'#line 1 "{path}"']
    for n, line in enumerate(lines):
        if n in at:
            _, before, after = HOOKS[at[n]]
            if before:
                out += before + [f'#line {n + 1} "{path}"']
            out.append(line)
            if after:
                out += after + [f'#line {n + 2} "{path}"']
        else:
            out.append(line)
    sys.stdout.write("\n".join(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
