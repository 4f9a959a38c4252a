"""Print the compiler/linker flags needed to build the reference's ATen CPU path against the
installed torch (test infrastructure only; used by oracle/Makefile's `ref` target)."""
import os
import sys
import sysconfig

import torch
from torch.utils import cpp_extension


def cflags() -> str:
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"]]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return " ".join([f"-I{p}" for p in incs] + [f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
                                                  "-DTORCH_EXTENSION_NAME=ref_lstm", "-w"])


def ldflags() -> str:
    lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    return f"-L{lib} -Wl,-rpath,{lib} -ltorch -ltorch_cpu -lc10"


if __name__ == "__main__":
    print(cflags() if sys.argv[1] == "cflags" else ldflags())
