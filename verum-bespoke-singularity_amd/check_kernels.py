#!/usr/bin/env python3
"""Build-time check of the gfx950 code objects this package compiles.

    python3 check_kernels.py build/*.o

For every object built from csrc/*.hip (its .hip_fatbin section unbundled
for gfx950 with the ROCm LLVM tools):

* the kernels whose loads the compiler does not track -- the LDS-DMA and
  inline-assembly loads of k_mvl, k_mvr, k_mvbr4, k_mvbr6 and k_checksum,
  each waited for by an explicit vmcnt count (csrc/vbs_lds_dma.h) -- spill
  no vector register and use no scratch: the code object metadata must show
  .vgpr_spill_count and .private_segment_fixed_size of 0 (a spill's scratch
  load or store would be counted by the same vmcnt and throw the
  hand-counted waits off, and a copy of a destination register made before
  its wait would hold stale data). Scalar registers spilled into lanes of a
  vector register (v_writelane / v_readlane, no memory: the case whenever
  .sgpr_spill_count is not 0 while the scratch size is) are allowed;
* M0 is written only by the LDS-DMA sequence of csrc/vbs_lds_dma.h and
  csrc/vbs_kern_checksum.hip (s_mov_b32 m0, sN; s_nop 0; global_load_lds_*),
  and read by nothing else: those inline-assembly blocks set M0 without
  declaring it (M0 is a reserved register the compiler does not save), so
  any other use of M0 by compiler-generated code in the same kernel would be
  overwritten behind its back.

Exits 1 with the offending kernels listed; 0 when every object passes.
"""
import os
import re
import subprocess
import sys
import tempfile

LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def code_object(obj, tmp):
    fb = os.path.join(tmp, os.path.basename(obj) + ".fatbin")
    co = os.path.join(tmp, os.path.basename(obj) + ".co")
    subprocess.run(["objcopy", f"--dump-section=.hip_fatbin={fb}", obj], check=True,
                   capture_output=True)
    subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={fb}",
                    f"--targets={TARGET}", f"--output={co}"], check=True, capture_output=True)
    return co


HAND_WAITED = re.compile(r"k_mvl|k_mvr|k_mvbr4|k_mvbr6|k_checksum")


def metadata_problems(co):
    notes = subprocess.run([f"{LLVM}/llvm-readelf", "--notes", co], check=True,
                           capture_output=True, text=True).stdout
    bad, cur = [], {}
    for line in notes.splitlines():
        m = re.match(r"\s*-?\s*\.(name|vgpr_spill_count|sgpr_spill_count|"
                     r"private_segment_fixed_size):\s+(\S+)", line)
        if not m:
            continue
        key, val = m.group(1), m.group(2)
        cur[key] = val
        if all(k in cur for k in ("name", "vgpr_spill_count", "sgpr_spill_count",
                                  "private_segment_fixed_size")):
            if HAND_WAITED.search(cur["name"]) and (
                    cur["vgpr_spill_count"], cur["private_segment_fixed_size"]) != ("0", "0"):
                bad.append(f"{cur['name']}: vgpr spills {cur['vgpr_spill_count']}, sgpr spills "
                           f"{cur['sgpr_spill_count']}, scratch {cur['private_segment_fixed_size']}")
            cur = {}
    return bad


def m0_problems(co):
    dis = subprocess.run([f"{LLVM}/llvm-objdump", "-d", co], check=True, capture_output=True,
                         text=True).stdout
    bad, kernel, ins = [], "?", []
    for line in dis.splitlines():
        k = re.match(r"^[0-9a-f]+ <(.+)>:", line)
        if k:
            kernel = k.group(1)
            continue
        m = re.match(r"^\s+(\S.*?)\s*//", line)
        if m:
            ins.append((kernel, m.group(1)))
    for i, (kern, text) in enumerate(ins):
        if not re.search(r"\bm0\b", text):
            continue
        ok = (re.match(r"s_mov_b32 m0, s\d+$", text) and i + 2 < len(ins) and
              ins[i + 1][1] == "s_nop 0" and ins[i + 2][1].startswith("global_load_lds_dword"))
        if not ok:
            bad.append(f"{kern}: {text}")
    return bad


def main(objs):
    if not os.path.exists(f"{LLVM}/clang-offload-bundler"):
        print("check_kernels: ROCm LLVM tools not found; skipped")
        return 0
    problems = []
    with tempfile.TemporaryDirectory() as tmp:
        for obj in objs:
            co = code_object(obj, tmp)
            problems += [f"{os.path.basename(obj)}: {p}" for p in metadata_problems(co)]
            problems += [f"{os.path.basename(obj)}: M0 outside the DMA sequence: {p}"
                         for p in m0_problems(co)]
    for p in problems:
        print(p)
    print(f"check_kernels: {len(objs)} objects, {len(problems)} problems")
    return 1 if problems else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
