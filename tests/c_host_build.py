"""Builds tests/c_host/drop_in.c, the plain C host of the library (no Python
or PyTorch in its process), with gcc against include/pbsample.h and
promptboot_amd/libpbsample.so."""
import pathlib
import subprocess

ROOT = pathlib.Path(__file__).resolve().parents[1]
ROCM = pathlib.Path("/opt/rocm")


def build_drop_in(out_dir: pathlib.Path) -> pathlib.Path:
    exe = out_dir / "drop_in"
    lib_dir = ROOT / "promptboot_amd"
    cmd = ["gcc", "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROCM / 'include'}", f"-I{ROOT / 'include'}", str(ROOT / "tests" / "c_host" / "drop_in.c"),
           f"-L{lib_dir}", "-lpbsample", f"-L{ROCM / 'lib'}", "-lamdhip64",
           f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe
