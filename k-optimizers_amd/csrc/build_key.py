"""Build kaon_amd/_kaon_key*.so (kaon_key.cpp) in-tree with g++ against the
installed torch's headers and libraries: python build_key.py"""
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(os.path.dirname(HERE), "kaon_amd", "_kaon_key" + sysconfig.get_config_var("EXT_SUFFIX"))


def build() -> str:
    import torch
    import torch.utils.cpp_extension as cx

    libdir = cx.library_paths()[0]
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}"]
    cmd += [f"-I{p}" for p in cx.include_paths()] + [f"-I{sysconfig.get_paths()['include']}"]
    cmd += [os.path.join(HERE, "kaon_key.cpp"), f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
            f"-Wl,-rpath,{libdir}", "-o", OUT]
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    print(build())
    sys.exit(0)
