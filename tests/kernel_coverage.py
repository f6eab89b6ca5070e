"""Kernel coverage of the GPU test suite.

Lists every kernel instantiation compiled into the library's device code (the
kernel descriptors of the gfx950 code objects inside quant-lib_amd/csrc/*.o,
read with the ROCm LLVM tools) and checks them against a rocprofv3 kernel trace
of `pytest -m gpu` taken with mangled names: a kernel that no test launched is
a dispatch branch whose results nothing checks.  Prints a per-family table and
the kernels never launched; exits 1 if there are any.

    (cd quant-lib_amd && make)
    rocprofv3 --kernel-trace -M -f csv -d OUT -o cov -- python3 -m pytest tests -m gpu -q
    python3 tests/kernel_coverage.py OUT/cov_kernel_trace.csv

Not collected by pytest (no test_ prefix): it needs the trace of a whole GPU run.
"""
import collections
import csv
import pathlib
import re
import subprocess
import sys
import tempfile

ROOT = pathlib.Path(__file__).resolve().parent.parent
CSRC = ROOT / "quant-lib_amd" / "csrc"
LLVM = pathlib.Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def compiled_kernels():
    """{mangled kernel name: source file stem} over the .o files built from .hip sources."""
    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        for hip in sorted(CSRC.glob("*.hip")):
            obj = hip.with_suffix(".o")
            if not obj.exists():
                raise SystemExit(f"{obj} is missing: build the library first")
            fat, co = pathlib.Path(tmp) / "fatbin", pathlib.Path(tmp) / "co.elf"
            subprocess.run([LLVM / "llvm-objcopy", f"--dump-section=.hip_fatbin={fat}", obj,
                            pathlib.Path(tmp) / "host.o"], check=True)
            subprocess.run([LLVM / "clang-offload-bundler", "--unbundle", "--type=o",
                            f"--input={fat}", f"--targets={TARGET}", f"--output={co}"], check=True)
            syms = subprocess.run([LLVM / "llvm-readelf", "--syms", co], check=True,
                                  capture_output=True, text=True).stdout
            for line in syms.splitlines():
                f = line.split()
                if len(f) >= 8 and f[7].endswith(".kd"):
                    out[f[7][:-3]] = hip.stem
    return out


def launched_kernels(trace_csv):
    counts = collections.Counter()
    with open(trace_csv, newline="") as fh:
        for row in csv.DictReader(fh):
            name = row["Kernel_Name"]
            counts[name[:-3] if name.endswith(".kd") else name] += 1
    return counts


def family(mangled):
    """Template name of an Itanium-mangled kernel (anonymous namespace or global)."""
    m = re.match(r"_ZN12_GLOBAL__N_1(\d+)", mangled) or re.match(r"_Z(\d+)", mangled)
    if not m:
        return mangled
    n = int(m.group(1))
    return mangled[m.end():m.end() + n]


def main(argv):
    if len(argv) != 2:
        raise SystemExit(__doc__)
    compiled = compiled_kernels()
    launched = launched_kernels(argv[1])
    fam = collections.defaultdict(lambda: [0, 0, 0])
    never = []
    for name, src in sorted(compiled.items()):
        key = (src, family(name))
        fam[key][0] += 1
        if launched.get(name, 0):
            fam[key][1] += 1
            fam[key][2] += launched[name]
        else:
            never.append(name)
    print("| source | kernel template | instantiations | launched by the suite | launches |")
    print("|---|---|---|---|---|")
    for (src, f), (n, hit, calls) in sorted(fam.items()):
        print(f"| {src}.hip | {f} | {n} | {hit} | {calls} |")
    total_hit = sum(v[1] for v in fam.values())
    print(f"\n{len(compiled)} kernel instantiations compiled, {total_hit} launched, "
          f"{len(never)} never launched")
    for name in never:
        print("never launched:", name)
    return 1 if never else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
