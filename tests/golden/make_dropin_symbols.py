"""Writes tests/golden/dropin_symbols.txt: the mangled C++ symbols that code compiled
against the reference's own headers needs from the library that replaces the GPU half of
the quantized path (the four conv_quant_detail launchers, cuda_kernels.cu:1465-1499) and
from the harness (verify_tensors, benchmark_cuda_op).

    python tests/golden/make_dropin_symbols.py      # needs /root/reference and g++

A probe translation unit that takes the address of each function is compiled with
-I/root/reference/src; its undefined symbols are the drop-in ABI.
"""
import subprocess
import tempfile
from pathlib import Path

PROBE = r'''
#include "conv_types.h"
void* dropin_probe[] = {
  (void*)&conv_quant_detail::launch_fprop_nhwc_qi32_u8,
  (void*)&conv_quant_detail::launch_fprop_nhwc_qi32_s5,
  (void*)&conv_quant_detail::launch_block_fprop_nhwc_qi32_u8,
  (void*)&conv_quant_detail::launch_block_fprop_nhwc_qi32_s5,
  (void*)&verify_tensors,
  (void*)&benchmark_cuda_op,
};
'''


def main(ref: str = "/root/reference") -> None:
    with tempfile.TemporaryDirectory() as d:
        src = Path(d) / "probe.cpp"
        obj = Path(d) / "probe.o"
        src.write_text(PROBE)
        subprocess.run(["g++", "-std=c++17", f"-I{ref}/src", "-c", str(src), "-o", str(obj)], check=True)
        out = subprocess.run(["nm", "-u", str(obj)], check=True, capture_output=True, text=True).stdout
    syms = sorted(ln.split()[-1] for ln in out.splitlines() if ln.strip())
    dest = Path(__file__).resolve().parent / "dropin_symbols.txt"
    dest.write_text("\n".join(syms) + "\n")
    print(dest, len(syms))


if __name__ == "__main__":
    main()
