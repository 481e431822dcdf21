"""In-tree build of libnanoserve_amd.so (hipcc, gfx950) through the Makefile beside this file."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def build(force: bool = True, jobs: int = 8) -> str:
    """Compile every HIP source for gfx950 and link libnanoserve_amd.so. With ``force`` the
    sources are recompiled even when the library is up to date."""
    cmd = ["make", "-s", "-C", HERE, f"-j{jobs}", "all"]
    if force:
        cmd.insert(2, "-B")
    subprocess.run(cmd, check=True)
    return os.path.join(HERE, "libnanoserve_amd.so")


if __name__ == "__main__":
    print(build())
