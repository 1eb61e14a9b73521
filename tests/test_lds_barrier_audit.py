"""Static check of the built gfx950 code: no workgroup barrier is reached
while this wave's LDS reads may still be outstanding.

On gfx950 the compiler does not make ``s_barrier`` wait for the wave's
earlier LDS reads (the target's barrier backs off instead), and across a
loop's back edge the barrier's fence does not add that wait either. A read
issued before a barrier whose value is first used after it can then return
after another wave, released by the barrier, has rewritten the word. The
per-tile depth sort had exactly this race (lane masks cleared over exchange
words other waves were still reading) until each wave waited for its reads
(``lds_reads_done``) before that barrier.

The check compiles every source to gfx950 assembly with the library's own
flags and runs a dataflow pass over each kernel's control-flow graph: the
number of LDS reads (``ds_read*``/``ds_load*``) issued since the last
``s_waitcnt lgkmcnt(n)`` that covers them, maximised over paths, must be
zero at every ``s_barrier``. It is pinned by a planted kernel with the race
(flagged) and the same kernel with the wait (not flagged). CPU only: hipcc
cross-compiles here.
"""

from __future__ import annotations

import importlib.util
import re
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _build_module():
    spec = importlib.util.spec_from_file_location("_mg_build_audit",
                                                  ROOT / "metal-gauss_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _assemble(src: Path, out: Path, name: str) -> Path:
    b = _build_module()
    cmd = [b.hipcc(), *b.CFLAGS, *b.FILE_FLAGS.get(name, []), f"-I{b.CSRC}",
           "--offload-device-only", "-S", str(src), "-o", str(out)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src.name}:\n{p.stderr}")
    return out


def _functions(path: Path) -> dict[str, list[str]]:
    funcs, cur = {}, None
    for line in path.read_text().splitlines():
        s = line.split(";")[0].strip()
        m = re.match(r"^([A-Za-z_]\w*):$", s)
        if m and not s.startswith(".L"):
            cur = m.group(1)
            funcs[cur] = []
            continue
        if cur is None or not s:
            continue
        if s.startswith(".Lfunc_end"):
            cur = None
            continue
        if s.startswith(".") and not re.match(r"^\.LBB\w+:$", s):
            continue
        funcs[cur].append(s)
    return funcs


def _blocks(body):
    blocks, cur = [], {"label": None, "ins": []}
    for s in body:
        if re.match(r"^\.LBB\w+:$", s):
            if cur["ins"] or cur["label"]:
                blocks.append(cur)
            cur = {"label": s[:-1], "ins": []}
            continue
        cur["ins"].append(s)
        op = s.split()[0]
        if op.startswith("s_cbranch") or op in ("s_branch", "s_endpgm") or op.startswith("s_setpc"):
            blocks.append(cur)
            cur = {"label": None, "ins": []}
    if cur["ins"] or cur["label"]:
        blocks.append(cur)
    return blocks


def pending_reads_at_barriers(body) -> list[int]:
    """For each s_barrier of one function (in order), the largest number of
    LDS reads that may be outstanding when it is reached."""
    blocks = _blocks(body)
    if not blocks:
        return []
    index = {b["label"]: i for i, b in enumerate(blocks) if b["label"]}
    succ = []
    for i, b in enumerate(blocks):
        last = b["ins"][-1] if b["ins"] else ""
        op = last.split()[0] if last else ""
        if op == "s_branch":
            nxt = [index[last.split()[1]]]
        elif op.startswith("s_cbranch"):
            nxt = [index[last.split()[1]], i + 1]
        elif op in ("s_endpgm",) or op.startswith("s_setpc"):
            nxt = []
        else:
            nxt = [i + 1]
        succ.append([j for j in nxt if j < len(blocks)])
    entry = [0] * len(blocks)
    reached = [False] * len(blocks)
    reached[0] = True
    at_barrier: dict[tuple[int, int], int] = {}
    changed = True
    while changed:
        changed = False
        for i, b in enumerate(blocks):
            if not reached[i]:
                continue
            p = entry[i]
            for k, s in enumerate(b["ins"]):
                op = s.split()[0]
                if op.startswith("ds_read") or op.startswith("ds_load"):
                    p = min(p + 1, 63)
                elif op == "s_waitcnt" and "lgkmcnt(" in s:
                    p = min(p, int(re.search(r"lgkmcnt\((\d+)\)", s).group(1)))
                elif op == "s_barrier":
                    at_barrier[(i, k)] = max(at_barrier.get((i, k), 0), p)
            for j in succ[i]:
                if not reached[j] or p > entry[j]:
                    reached[j] = True
                    entry[j] = max(entry[j], p)
                    changed = True
    return [at_barrier[key] for key in sorted(at_barrier)]


@pytest.fixture(scope="module")
def assembly(tmp_path_factory):
    b = _build_module()
    out = tmp_path_factory.mktemp("isa")
    with ThreadPoolExecutor(max_workers=8) as ex:
        futs = {s: ex.submit(_assemble, b.CSRC / s, out / (Path(s).stem + ".s"), s)
                for s in b.SOURCES}
        return {s: f.result() for s, f in futs.items()}


def test_no_barrier_waits_on_outstanding_lds_reads(assembly):
    bad, kernels, barriers = [], 0, 0
    for src, path in assembly.items():
        for fn, body in _functions(path).items():
            counts = pending_reads_at_barriers(body)
            if counts:
                kernels += 1
                barriers += len(counts)
            if any(counts):
                bad.append(f"{src}: {fn}: {counts}")
    print(f"{kernels} kernels with barriers, {barriers} barriers checked")
    assert kernels > 40 and barriers > 150, (kernels, barriers)
    assert not bad, "barriers reached with LDS reads outstanding:\n" + "\n".join(bad)


# The hazard in its smallest form: each iteration a wave reads a word that
# another wave wrote, and first uses the value after the next iteration's
# barrier, behind which the word is rewritten. WAIT is empty (the race) or a
# wait for the wave's LDS reads before that barrier (the fix).
PLANTED = r"""
#include <hip/hip_runtime.h>
__device__ __forceinline__ void lds_reads_done() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}
extern "C" __global__ void __launch_bounds__(256) planted(const float *in, float *out, int n) {
    __shared__ float s[256];
    float v = 0.f;
    for (int it = 0; it < n; ++it) {
        WAIT
        __syncthreads();
        s[threadIdx.x] = in[it * 256 + threadIdx.x] + v;
        __syncthreads();
        v = s[255 - threadIdx.x];
    }
    out[threadIdx.x] = v;
}
"""


@pytest.mark.parametrize("wait,flagged", [("", True), ("lds_reads_done();", False)])
def test_the_check_flags_a_read_first_used_after_the_next_barrier(tmp_path, wait, flagged):
    """The planted mistake (a loop whose LDS read is used after the next
    barrier) is flagged at that barrier; with the wave's reads waited for
    before it, it is not."""
    src = tmp_path / "planted.hip"
    src.write_text(PLANTED.replace("WAIT", wait))
    funcs = _functions(_assemble(src, tmp_path / "planted.s", "planted.hip"))
    assert "planted" in funcs
    assert any(pending_reads_at_barriers(funcs["planted"])) == flagged
