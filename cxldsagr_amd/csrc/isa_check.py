"""Build check: no matrix instruction in an EXEC-masked block that the GPU runs
with EXEC = 0.

MFMA instructions ignore the EXEC mask: all 64 lanes compute and write the
destination whatever EXEC holds. A branch on a value the compiler cannot prove
wave-uniform (``threadIdx.x >> 6`` is such a value) is lowered to EXEC masking:
``s_and_saveexec`` opens the taken side, ``s_andn2_saveexec`` / ``s_or_saveexec``
/ ``s_xor_b64 exec`` switch to the other side, ``s_or_b64 exec, exec`` closes
the region. For a wave that takes one side, the other side runs with EXEC = 0
unless an ``s_cbranch_execz`` skips it, and the compiler drops that skip for
short blocks. An MFMA in such a block then overwrites its accumulator with the
other side's operands. (A 16x16x32 MFMA in a two-way ``if`` on ``wave & 1``
produced wrong row sums for every odd wave in exactly this way; making the
condition ``__builtin_amdgcn_readfirstlane(wave) & 1`` turns it into a scalar
branch.)

This module compiles each source to gfx950 assembly with the library's flags
and reports every MFMA that sits in a masked side with no EXEC-zero skip. It
also reports every kernel that spills to scratch memory beyond the spills
listed in KNOWN_SPILLS: the kernels' occupancy and speed are tuned to their
register counts (the layer prologue to three work-groups per CU at 168
registers), and a spill is the first sign that a change pushed one over.
Usage: ``python -m cxldsagr_amd.csrc.isa_check`` (exit status 1 on a finding).
"""

import re
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

from cxldsagr_amd.csrc import build

_LABEL = re.compile(r"^(_Z[\w.$]+):")
_KERNEL = re.compile(r"^\s*\.amdhsa_kernel\s+(\S+)")
_SCRATCH = re.compile(r"^\s*\.amdhsa_private_segment_fixed_size\s+(\d+)")

# Spills accepted as they are: (substring of the kernel symbol, bytes per lane).
# topk_rows<17> keeps 68 scores per thread in registers for rows of up to
# 69,632 columns (configs 1+2 of the unfused top-k) and spills 28 bytes.
KNOWN_SPILLS = {"topk_rowsILi17E": 28}


def unguarded_mfma(asm):
    """``[(function, line, side_start_line), ...]`` for each MFMA of ``asm``
    (gfx9 assembly text) inside an EXEC-masked side that no ``s_cbranch_execz``
    skips."""
    found = []
    function, stack = None, []
    for number, raw in enumerate(asm.splitlines(), 1):
        line = raw.strip()
        label = _LABEL.match(line)
        if label:
            function, stack = label.group(1), []
        if not line or line.startswith((";", ".")) or line.endswith(":"):
            continue
        if line.startswith("s_and_saveexec_b64"):
            stack.append({"skip": False, "open": True, "start": number})
            continue
        if line.startswith(("s_andn2_saveexec_b64", "s_or_saveexec_b64", "s_xor_b64 exec, exec")):
            if stack:
                stack[-1].update(skip=False, open=True, start=number)
            continue
        if line.startswith("s_or_b64 exec, exec"):
            if stack:
                stack.pop()
            continue
        if line.startswith("s_cbranch_execz"):
            if stack and stack[-1]["open"]:
                stack[-1]["skip"] = True
            continue
        if stack and not line.startswith("s_"):
            # The side's first vector or memory instruction: a skip must come before it.
            stack[-1]["open"] = False
        if line.startswith("v_mfma") and stack and not stack[-1]["skip"]:
            found.append((function, number, stack[-1]["start"]))
    return found


def scratch_bytes(asm):
    """``{kernel symbol: scratch bytes per lane}`` for each kernel of ``asm``
    with a nonzero private segment."""
    found, kernel = {}, None
    for raw in asm.splitlines():
        m = _KERNEL.match(raw)
        if m:
            kernel = m.group(1)
            continue
        m = _SCRATCH.match(raw)
        if m and kernel and int(m.group(1)):
            found[kernel] = int(m.group(1))
    return found


def unknown_spills(found):
    """The entries of ``found`` (``scratch_bytes``) that KNOWN_SPILLS does not list."""
    return {kernel: size for kernel, size in found.items()
            if not any(key in kernel and size == known for key, known in KNOWN_SPILLS.items())}


def device_asm(source, out_dir):
    """gfx950 assembly of one source with the library's compile flags."""
    out = Path(out_dir) / (Path(source).stem + ".s")
    cmd = [build.hipcc(), *build.FLAGS, *build.SOURCE_FLAGS.get(Path(source).name, []),
           "--cuda-device-only", "-S", str(source), "-o", str(out)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {Path(source).name}:\n{result.stderr}")
    return out.read_text()


def _texts(sources):
    with tempfile.TemporaryDirectory() as tmp, ThreadPoolExecutor(max_workers=8) as pool:
        return list(pool.map(lambda s: device_asm(s, tmp), sources))


def analyse(sources=None):
    """``(mfma, spills)``: ``{source name: unguarded_mfma findings}`` and
    ``{source name: {kernel: bytes}}`` of the spills KNOWN_SPILLS does not
    list, each holding only the sources with a finding."""
    sources = list(sources or build.sources())
    mfma, spills = {}, {}
    for source, text in zip(sources, _texts(sources)):
        findings = unguarded_mfma(text)
        if findings:
            mfma[Path(source).name] = findings
        extra = unknown_spills(scratch_bytes(text))
        if extra:
            spills[Path(source).name] = extra
    return mfma, spills


def check(sources=None):
    """``{source name: findings}`` for every source with an unguarded MFMA."""
    return analyse(sources)[0]


if __name__ == "__main__":
    problems, spills = analyse()
    for name, findings in problems.items():
        for function, line, start in findings[:5]:
            print(f"{name}: {function}: MFMA at assembly line {line} in the masked side "
                  f"opened at line {start}, with no s_cbranch_execz skip")
    for name, kernels in spills.items():
        for kernel, size in kernels.items():
            print(f"{name}: {kernel}: {size} bytes of scratch per lane")
    sys.exit(1 if problems or spills else 0)
