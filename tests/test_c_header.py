"""The C ABI from C: include/mi_attn.h compiles as C99 with warnings as errors,
links against the library, and the host-side entry points behave as declared
(version, status strings, argument validation before any launch).  No GPU call
is made: every compute entry point here fails validation first."""
import os
import shutil
import subprocess

import pytest

from gpt_from_scratch_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

C_SOURCE = r"""
#include <stdio.h>
#include <string.h>
#include "mi_attn.h"

int main(void) {
  if ((mi_version() >> 16) != 2) return 1;
  if (strcmp(mi_status_str(MI_OK), "ok") != 0) return 2;
  const int64_t st[4] = {0, 0, 64, 1};
  char dummy[16];
  /* unknown dtype: rejected before anything is launched */
  if (mi_attn_fwd((mi_dtype)7, 1, 1, 64, 64, 1, 0.125f, dummy, st, dummy, st, dummy, st,
                  dummy, st, (float*)dummy, NULL) != MI_ERR_INVALID_ARGUMENT) return 3;
  if (strstr(mi_last_error(), "dtype") == NULL) return 4;
  /* RMSNorm workspace query and an invalid weight dtype */
  if (mi_rmsnorm_bwd_workspace(4, 768) != 768) return 5;
  if (mi_rmsnorm_fwd(MI_BF16, MI_F16, 4, 768, 1e-6f, dummy, 768, dummy, dummy, 768,
                     (float*)dummy, NULL) != MI_ERR_INVALID_ARGUMENT) return 6;
  if (mi_adamw_workspace() < 2) return 7;
  printf("ok %d\n", mi_version());
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_header_is_c99_and_links(tmp_path):
    _lib.lib()  # the library must exist (built by build())
    src = tmp_path / "abi.c"
    src.write_text(C_SOURCE)
    exe = tmp_path / "abi"
    libdir = os.path.dirname(_lib.LIB_PATH)
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           str(src), "-o", str(exe), "-L", libdir, "-l:libmi_attn.so", f"-Wl,-rpath,{libdir}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # the library's HIP runtime dependency resolves through ROCm's lib directory
    env = dict(os.environ)
    env["LD_LIBRARY_PATH"] = ":".join(p for p in ("/opt/rocm/lib", env.get("LD_LIBRARY_PATH", ""))
                                      if p)
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert r.stdout.startswith("ok ")
