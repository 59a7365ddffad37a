"""include/llb_backend_hip.h is a backend the reference host's contract header accepts: a translation unit
that includes it and then host/llb_backend.h (the reference refuses to compile without a backend that
defines LLB_LAUNCH, host/llb_backend.h:48-50) compiles warning-free as C11 and links against the in-tree
library, with every name of the contract (host/llb_backend.h:8-41) used as the reference's chains use
it: LLB_LAUNCH / LLB_LAUNCH_SM with argument addresses of a u32, a float, an llb_dptr and a by-value
struct, each returning bool; llb_alloc_zero returning llb_dptr; llb_zero / llb_copy / llb_write /
llb_read / llb_sync returning bool; llb_dev of a host pointer. Nothing runs: no GPU is needed. On the GPU
the C driver (moe_layer_drv, tests/test_driver.py) runs through these macros."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_HOST = "/root/reference/host"
LIB_DIR = os.path.join(ROOT, "eureka-engine_amd")

USER = r"""
#include "llb_backend_hip.h"
#include "%s/llb_backend.h"

typedef struct { llb_dptr q; unsigned n; float s; } Cat;  /* a by-value struct argument (Q8Cat-like) */

#define SAME(a, T) _Static_assert(_Generic((a), T: 1, default: 0), #a " has the contract's type")

bool chain(void* k, llb_dptr buf, unsigned n, float eps, void* host, size_t bytes) {
  Cat c = {buf, n, eps};
  llb_dptr p = llb_alloc_zero(bytes);
  SAME(LLB_LAUNCH(k, 1, 1, 64, &buf, &n), bool);
  SAME(LLB_LAUNCH_SM(k, 1, 1, 64, 4096, &buf), bool);
  SAME(llb_alloc_zero(bytes), llb_dptr);
  SAME(llb_dev(host), llb_dptr);
  return p != 0 && LLB_LAUNCH(k, (n + 255) / 256, 2, 256, &buf, &n, &eps, &c) &&
         LLB_LAUNCH_SM(k, 1, n, 1024, 8192, &p, &c) && llb_zero(p + 4096 * 4, 16) && llb_copy(p, buf, 16) &&
         llb_write(p, host, 16) && llb_read(host, p, 16) && llb_sync() && llb_dev(host) != 0;
}
int main(void) { return chain(0, 0, 0, 0.f, 0, 0) ? 0 : 1; }
"""


def _gcc(src, tmp_path, *extra):
    f = tmp_path / "user.c"
    f.write_text(src)
    return subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
                           str(f), *extra], capture_output=True, text=True, timeout=120)


needs_ref = pytest.mark.skipif(not os.path.exists(os.path.join(REF_HOST, "llb_backend.h")),
                               reason="the reference tree is not present (the GPU box has none)")


@needs_ref
def test_reference_contract_header_accepts_the_hip_backend(tmp_path):
    r = _gcc(USER % REF_HOST, tmp_path, "-fsyntax-only")
    assert r.returncode == 0, r.stderr


@needs_ref
def test_reference_contract_header_refuses_no_backend(tmp_path):
    r = _gcc('#include "%s/llb_backend.h"\nint main(void) { return 0; }\n' % REF_HOST, tmp_path, "-fsyntax-only")
    assert r.returncode != 0 and "include a backend" in r.stderr


@needs_ref
def test_backend_user_links_against_the_library(tmp_path):
    if not os.path.exists(os.path.join(LIB_DIR, "libeureka_moe.so")):
        pytest.fail("libeureka_moe.so is not built (eureka-engine_amd/build.sh)")
    r = _gcc(USER % REF_HOST, tmp_path, "-o", str(tmp_path / "user"), "-L", LIB_DIR, "-leureka_moe")
    assert r.returncode == 0, r.stderr


def test_launch_argument_count_is_the_macro_arity(tmp_path):
    """the macro hands the library the number of argument addresses it was given (no reference needed):
    a stub llb_hip_launch records na and the address of each argument."""
    src = r"""
#include "llb_backend_hip.h"
#include <stdio.h>
static unsigned got_na, got_sm, got_gy; static void** got_a;
int llb_hip_launch(void* fn, uint32_t gx, uint32_t gy, uint32_t bx, uint32_t sm, void** args, uint32_t na) {
  (void)fn; (void)gx; (void)bx; got_na = na; got_sm = sm; got_gy = gy; got_a = args; return 0; }
int main(void) {
  unsigned n = 7; float e = 2.f; llb_dptr p = 9;
  if (!LLB_LAUNCH((void*)1, 1, 3, 64, &p, &n, &e) || got_na != 3 || got_sm != 0 || got_gy != 3) return 1;
  if (got_a[0] != (void*)&p || got_a[2] != (void*)&e) return 2;
  if (!LLB_LAUNCH_SM((void*)1, 1, 1, 64, 512, &n) || got_na != 1 || got_sm != 512) return 3;
  return 0;
}
"""
    r = _gcc(src, tmp_path, "-o", str(tmp_path / "t"))
    assert r.returncode == 0, r.stderr
    assert subprocess.run([str(tmp_path / "t")], timeout=30).returncode == 0
