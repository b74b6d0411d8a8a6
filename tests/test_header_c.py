"""include/venturi_ops.h as a C and a C++ runtime would use it (no GPU): the header
compiles on its own as C11 and C++17 with warnings as errors, a program that
calls the library links against libventuri_ops.so, and at run time it reads the
identity, sizes a workspace and gets the documented rejection (-1 and a message)
for invalid arguments before any HIP call."""

import shutil
import subprocess

import pytest

from venturi_amd import native

from test_abi import HEADER

PROGRAM = r"""
#include "venturi_ops.h"
#include <stdio.h>
#include <string.h>

int main(void) {
    if (venturi_blocks_abi() != 18 || venturi_blocks_arch() != 950) return 1;
    if (venturi_q8_dp4a_bytes(3, 100, 2) != (uint64_t)(3 * 4 * 36 * 2)) return 2;
    /* tokens = 0 is invalid: rejected on the host, nothing is launched. */
    if (venturi_q8_head_run(NULL, NULL, NULL, NULL, 0, 1, 128, 128, 0, NULL) != -1) return 3;
    const char* why = venturi_blocks_error();
    if (why == NULL || strlen(why) == 0) return 4;
    printf("ok %s\n", why);
    return 0;
}
"""


@pytest.mark.parametrize("compiler,std,source", [("gcc", "-std=c11", "consumer.c"), ("g++", "-std=c++17", "consumer.cpp")])
def test_header_compiles_links_and_rejects(tmp_path, compiler, std, source):
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} is not installed")
    lib = native.DEFAULT_LIBRARY
    if not lib.exists():
        pytest.skip("libventuri_ops.so is not built")
    (tmp_path / source).write_text(PROGRAM)
    exe = tmp_path / "consumer"
    cmd = [compiler, std, "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{HEADER.parent}", str(tmp_path / source),
           f"-L{lib.parent}", "-lventuri_ops", f"-Wl,-rpath,{lib.parent}", "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, (run.returncode, run.stdout, run.stderr)
    assert run.stdout.startswith("ok ")
