"""The static library a Rust build.rs links (libbark_hip.a): a small C program
is linked against it with the system C compiler, amdhip64 and the C++ runtime
(the link line INTEGRATION.md gives), and exercises the device probe and the
error path of bark_hip_create without a GPU: no device index is valid here,
the call fails with a status code and a message, and no handle is returned."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB_A = ROOT / "bark3-wgpu_amd" / "libbark_hip.a"

PROGRAM = r"""
#include <stdio.h>
#include <string.h>
#include "bark_hip.h"
int main(void) {
  int n = bark_hip_device_count();
  BarkHip *h = (BarkHip *)0x1;
  int rc = bark_hip_create(n, 24, &h); /* device index n is never valid */
  const char *msg = bark_hip_last_error();
  printf("devices=%d rc=%d handle=%s msg=%s\n", n, rc, h ? "set" : "null", msg);
  if (h != 0 || rc >= 0 || msg == 0 || strlen(msg) == 0) return 1;
  if (bark_hip_create(0, 0, &h) != BARK_HIP_EINVAL) return 2; /* n_layers out of range */
  if (strstr(bark_hip_last_error(), "n_layers") == 0) return 3;
  bark_hip_destroy(0); /* a null handle is ignored */
  return 0;
}
"""


def test_static_library_links_into_a_c_program(tmp_path):
    if not LIB_A.exists():
        pytest.fail("libbark_hip.a is missing: run __graft_entry__.build() first")
    cc = shutil.which("gcc") or shutil.which("cc")
    assert cc, "no C compiler"
    src = tmp_path / "use_static.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "use_static"
    cmd = [cc, "-O1", f"-I{ROOT / 'include'}", str(src), "-o", str(exe), str(LIB_A), "-L/opt/rocm/lib",
           "-lamdhip64", "-lstdc++", "-lm", "-lpthread", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, f"exit {r.returncode}: {r.stdout}{r.stderr}"
    assert "handle=null" in r.stdout
