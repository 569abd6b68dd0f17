"""The grouped GEMM's ring schedule (ijah_amd/csrc/ring_schedule.h, used by chunk_gemm in moe_batch.hip), compiled
for the host and checked against an event simulation of the two rings: at every step the wait count the kernel uses
must leave both of that step's operands complete, and no ring slot may be refilled before its previous step consumed
it. Requests complete in issue order (the hardware's vector-memory counter rule the waits rely on).

The simulation shares no code with the header: it replays the issue order chunk_gemm follows (prologue A(0) B(0) ..
A(DA-1) B(DA-1) B(DA) .. B(DB-1); step s issues A(s + DA) and B(s + DB) after its wait and barrier) and records
where each request sits."""
import subprocess

import pytest

from conftest import ROOT

# (OA, OB, DA, DB): requests per A / B step and lead, for the shapes chunk_gemm instantiates (K < 6: DA 2, DB 5;
# K >= 6: DA 1, DB 3; OA 2 for the two-operand 128-row A, else 1; every B step is one request)
CONFIGS = [(2, 1, 2, 5), (1, 1, 2, 5), (2, 1, 1, 3), (1, 1, 1, 3)]
MAX_NS = 80


@pytest.fixture(scope="module")
def waits(tmp_path_factory):
    d = tmp_path_factory.mktemp("ring")
    src = d / "ring.cpp"
    lines = ['#include <cstdio>', '#include "ring_schedule.h"', "int main() {"]
    for oa, ob, da, db in CONFIGS:
        lines.append(f"  for (int ns = 1; ns <= {MAX_NS}; ns++) for (int t = 0; t < ns; t++) "
                     f'std::printf("{oa} {ob} {da} {db} %d %d %d\\n", ns, t, ijah::step_wait<{oa}, {ob}, {da}, {db}>(t, ns));')
    lines.append("  return 0;\n}")
    src.write_text("\n".join(lines))
    exe = d / "ring"
    subprocess.run(["g++", "-std=c++17", "-O1", f"-I{ROOT / 'ijah_amd' / 'csrc'}", str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    w = {}
    for line in out.splitlines():
        oa, ob, da, db, ns, t, n = map(int, line.split())
        w[(oa, ob, da, db, ns, t)] = n
    return w


def simulate(oa, ob, da, db, ns, wait):
    """Replays the issue order; returns the list of problems found (empty when the schedule is sound)."""
    issued = []  # request tags in issue order: ("A", step) or ("B", step), OA or OB entries per step
    slot_a, slot_b = {}, {}  # ring slot -> the step whose data it holds
    problems = []

    def issue(kind, j, now):
        ring, nslots = (slot_a, da + 1) if kind == "A" else (slot_b, db + 1)
        sl = j % nslots
        prev = ring.get(sl)
        if prev is not None and prev >= now:  # the previous occupant is consumed at its own step, before `now`
            problems.append(f"{kind}({j}) overwrites {kind}({prev}) in slot {sl} at step {now}")
        ring[sl] = j
        issued.extend([(kind, j)] * (oa if kind == "A" else ob))

    for j in range(min(db, ns)):  # prologue
        if j < da:
            issue("A", j, 0)
        issue("B", j, 0)
    for t in range(ns):
        done = len(issued) - wait(t)  # requests complete in issue order
        for kind in ("A", "B"):
            last = max(i for i, r in enumerate(issued) if r == (kind, t))
            if last >= done:
                problems.append(f"NS={ns} step {t}: {kind}({t}) may be outstanding after the wait")
        ring, nslots = (slot_a, da + 1), (slot_b, db + 1)
        if slot_a.get(t % (da + 1)) != t or slot_b.get(t % (db + 1)) != t:
            problems.append(f"NS={ns} step {t}: a ring slot does not hold step {t}")
        if t + da < ns:
            issue("A", t + da, t)
        if t + db < ns:
            issue("B", t + db, t)
    return problems


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: "OA{}_OB{}_DA{}_DB{}".format(*c))
def test_ring_schedule_waits_and_slots(waits, cfg):
    oa, ob, da, db = cfg
    for ns in range(1, MAX_NS + 1):
        probs = simulate(oa, ob, da, db, ns, lambda t: waits[(oa, ob, da, db, ns, t)])
        assert not probs, probs[:5]


def test_ring_schedule_waits_are_not_wasteful(waits):
    """In the steady state the wait leaves exactly the later step requests outstanding: a wait count one larger
    would let the step's own data be outstanding (so the count is the tightest sound one)."""
    oa, ob, da, db = CONFIGS[0]
    ns = MAX_NS
    probs = simulate(oa, ob, da, db, ns, lambda t: waits[(oa, ob, da, db, ns, t)] + 1)
    assert probs, "a looser wait was not caught: the simulation would not see a too-late wait"
