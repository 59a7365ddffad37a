"""The call-site code INTEGRATION.md gives a maintainer (the llb_moe_run replacement and the pf_moe
replacement) compiles as C11 against this library's headers and the reference's own host/llb_backend.h,
with stub declarations standing in for the reference host's names (u32, MoeL, gpu_mail, llb_scratch,
err_fail, ...), and links against the library. Nothing runs."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_HOST = "/root/reference/host"

STUBS = r"""
#include <stdint.h>
#include <stddef.h>
typedef uint32_t u32;
typedef uint64_t u64;
typedef struct { u32 d; } LlbShape;
typedef struct { llb_dptr g, u, d; const llb_dptr* pk; } MoeL;
typedef struct { const volatile u32* pt[64]; } Mail;
extern Mail* gpu_mail;
extern MoeL moe_l[64];
extern llb_dptr pf_x1;
extern float llb_cfg[4];
void err_fail(const char* msg);
void llb_scratch(llb_dptr* p, size_t* have, size_t n, const char* what);
"""


def blocks():
    src = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    cs = re.findall(r"```c\n(.*?)```", src, flags=re.S)
    run = next(c for c in cs if "llb_moe_run_hip" in c)
    pf = next(c for c in cs if "static void pf_moe" in c)
    return run, pf


def _cc(code, tmp_path, *extra):
    f = tmp_path / "site.c"
    f.write_text(code + "\nint main(void) { return 0; }\n")
    return subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-Wno-unused-function",
                           "-I", os.path.join(ROOT, "include"), *extra, str(f)],
                          capture_output=True, text=True, timeout=120)


def test_llb_moe_run_call_site_compiles(tmp_path):
    run, _ = blocks()
    head, body = run.split("\n", 1)  # the #include line first, then the stubs need llb_dptr
    r = _cc(head + "\n" + STUBS + body, tmp_path, "-fsyntax-only")
    assert r.returncode == 0, r.stderr


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_HOST, "llb_backend.h")),
                    reason="the reference tree is not present (the GPU box has none)")
def test_pf_moe_call_site_compiles_against_the_reference_contract(tmp_path):
    _, pf = blocks()
    lines = pf.split("\n")
    inc = "\n".join(l for l in lines if l.startswith("#include"))
    body = "\n".join(l for l in lines if not l.startswith("#include"))
    r = _cc(inc + "\n" + STUBS + body, tmp_path, "-I", REF_HOST, "-fsyntax-only")
    assert r.returncode == 0, r.stderr
