"""The library's C header and shared object serve a plain C host: the C host
program compiles warning-free as C11 and links against libpbsample.so (CPU;
running it needs the GPU, see test_gpu_c_host.py)."""
import pathlib

from tests.c_host_build import build_drop_in


def test_c_host_compiles_and_links(tmp_path: pathlib.Path):
    exe = build_drop_in(tmp_path)
    assert exe.exists() and exe.stat().st_size > 0
