"""Rewrites the library's kernel sources for the CPU emulation build
(tests/emu): the two LDS constructs plain C++ cannot express are mapped
onto the emulator's per-workgroup LDS block, and the AMDGPU-only function
attributes are dropped.  Everything else compiles as written against the
stand-in headers in tests/emu/include.

usage: prep.py SRC_DIR OUT_DIR"""
import os
import re
import sys


def rewrite(text):
    # extern __shared__ T name[];  ->  T* name = (T*)::emu::lds_base();
    text = re.sub(r"extern\s+__shared__\s+([\w\s]+?)\s+(\w+)\s*\[\s*\]\s*;",
                  r"\1* \2 = (\1*)::emu::lds_base();", text)
    # LDS byte addresses held as integers (the counters start at LDS address 0)
    names = re.findall(r"typedef\s+__attribute__\(\(address_space\(3\)\)\)\s+[\w\s]+?\s+(\w+)\s*;", text)
    text = re.sub(r"typedef\s+__attribute__\(\(address_space\(3\)\)\)\s+", "typedef ", text)
    for n in names:
        text = re.sub(r"\(%s\s*\*\)\s*\(uintptr_t\)\s*(\w+)" % n, r"(%s*)(::emu::lds_base() + (\1))" % n, text)
    text = re.sub(r"__attribute__\(\(amdgpu_waves_per_eu\([^)]*\)\)\)", "", text)
    return text


def main():
    src, out = sys.argv[1], sys.argv[2]
    os.makedirs(out, exist_ok=True)
    for name in sorted(os.listdir(src)):
        if not name.endswith((".hip", ".hpp", ".cpp")):
            continue
        with open(os.path.join(src, name)) as f:
            text = rewrite(f.read())
        dst = os.path.join(out, name[:-4] + ".cpp" if name.endswith(".hip") else name)
        old = None
        if os.path.exists(dst):
            with open(dst) as f:
                old = f.read()
        if old != text:
            with open(dst, "w") as f:
                f.write(text)


if __name__ == "__main__":
    main()
