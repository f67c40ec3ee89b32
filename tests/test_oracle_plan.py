"""The oracle's residency planner and planned-step semantics, pinned by hand-computed known answers.

The planner is a two-machine list schedule (include/bmx.h bmx_plan_policy; the reference's rule,
engine/kernels/nv2/nv2_host.cpp:1017-1030: the GPU starts at its base plus the hits, or at 0 with nothing resident;
the CPU lane starts at its base whenever it is eligible and something misses). Each case below was worked out by hand
from the rule's arithmetic; a planner with one plausible mistake planted (a strict comparison, the wrong sort
direction, the CPU base paid per expert, the GPU's resident term dropped, the CPU base paid only with the lane's first
expert, the GPU base paid with nothing resident) fails at least one of them."""
import numpy as np

import pytest

POL = dict(cpu_on=1, max_cpu=8, gpu_base_us=10.0, gpu_hit_us=1.0, gpu_admit_us=6.0, cpu_base_us=5.0,
           cpu_expert_us=4.0, cpu_token_us=2.0)

# (ex, res, cnt, ntok, npicks, rows, policy overrides, expected lanes)   V=0 A=1 H=2 C=3
CASES = [
    # default policy: residents V, every miss A
    ([1, 4, 7], [1, 0, 0], [2, 1, 1], 2, 4, True, None, [0, 1, 1]),
    # nothing resident: g = 0, c = 5. ex3 (cnt 3): ce = 5+4+4 = 13, max(13,0)=13 > max(5,6)=6 -> A (g 6); ex5 ce 9:
    # max(9,6)=9 <= max(5,12)=12 -> C (c 9); ex9 ce 13: max(13,6)=13 > max(9,12)=12 -> A
    ([3, 5, 9], [0, 0, 0], [3, 1, 1], 2, 5, True, {}, [1, 3, 1]),
    # two residents: g = 10+2 = 12, c = 5; ex3 ce 13: max(13,12)=13 <= max(5,18)=18 -> C (c 13); ex5 ce 17:
    # max(17,12)=17 <= max(13,18)=18 -> C (c 17); ex9 ce 21: max(21,12)=21 > max(17,18)=18 -> A
    ([2, 3, 5, 8, 9], [1, 0, 0, 1, 0], [1, 3, 1, 2, 1], 2, 8, True, {}, [0, 3, 3, 0, 1]),
    # max_cpu 1: ex3 A (as above), ex5 C, ex9 A (the lane is full)
    ([3, 5, 9], [0, 0, 0], [3, 1, 1], 2, 5, True, {"max_cpu": 1}, [1, 3, 1]),
    # order by picks descending, then expert ascending: ex9 (cnt 2) first: ce = 5+4+2 = 11 > max(5,6)=6 -> A (g 6);
    # ex3 ce 9: max(9,6)=9 <= max(5,12)=12 -> C (c 9); ex5 ce 13: max(13,6)=13 > max(9,12)=12 -> A
    ([3, 5, 9], [0, 0, 0], [1, 1, 2], 2, 4, True, {}, [3, 1, 1]),
    # tie goes to the CPU: one resident, g = 10, c = 0, ce = 10, gc = 0: max(10,10) = 10 <= max(0,10) = 10 -> C
    ([4, 6], [1, 0], [1, 1], 1, 2, True, {"cpu_base_us": 0.0, "cpu_expert_us": 10.0, "cpu_token_us": 0.0,
                                          "gpu_admit_us": 0.0, "gpu_hit_us": 0.0}, [0, 3]),
    # no rows with the request / too many picks / lane off: no CPU
    ([3, 5, 9], [0, 0, 0], [3, 1, 1], 2, 5, False, {}, [1, 1, 1]),
    ([3, 5, 9], [0, 0, 0], [3, 1, 1], 2, 65, True, {}, [1, 1, 1]),
    ([3, 5, 9], [0, 0, 0], [3, 1, 1], 2, 5, True, {"cpu_on": 0}, [1, 1, 1]),
    # home_single: single-pick misses of a multi-token call run from home (gpu_home 1). g = 0, c = 5: ex3 ce 13 > max(5,6)
    # -> A (g 6); ex5 home: ce 9, max(9,6)=9 > max(5,7)=7 -> H (g 7); ex9: max(9,7)=9 > max(5,8)=8 -> H
    ([3, 5, 9], [0, 0, 0], [3, 1, 1], 2, 5, True, {"home_single": 1, "gpu_home_us": 1.0}, [1, 2, 2]),
    # one token: home_single does not apply
    ([3, 5], [0, 0], [1, 1], 1, 2, True, {"home_single": 1, "gpu_home_us": 1.0, "cpu_on": 0}, [1, 1]),
    # the CPU base on both sides: a free CPU expert behind a base of 5 against a GPU admission of 1 with nothing resident:
    # g = 0, c = 5, ce = 5: max(5,0) = 5 <= max(5,1) = 5 -> C (paid only with the lane's first expert it would be
    # max(5,0) = 5 > max(0,1) = 1 -> A)
    ([6], [0], [1], 1, 1, True, {"cpu_expert_us": 0.0, "cpu_token_us": 0.0, "gpu_admit_us": 1.0}, [3]),
]


def run_case(planner, case):
    ex, res, cnt, ntok, npk, rows, over, _ = case
    pol = None if over is None else dict(POL, **over)
    return list(planner(np.array(ex), np.array(res), np.array(cnt), ntok, npk, rows, pol))


@pytest.mark.parametrize("i", range(len(CASES)))
def test_plan_known_answers(oracle, i):
    assert run_case(oracle.plan_lanes, CASES[i]) == CASES[i][-1]


def mutated(kind):
    """The planner's rule with one mistake planted."""
    def plan(ex, res, cnt, ntok, npicks, rows, policy=None):
        p = dict(dict(cpu_on=0, max_cpu=0, home_single=0, gpu_base_us=0.0, gpu_hit_us=0.0, gpu_home_us=0.0,
                      gpu_admit_us=0.0, cpu_base_us=0.0, cpu_expert_us=0.0, cpu_token_us=0.0), **(policy or {}))
        lanes = np.zeros(len(ex), np.int32)
        cpu_ok = p["cpu_on"] and rows and npicks <= 64 and ntok <= 8
        nres = int(np.sum(res != 0))
        key = (lambda u: (int(cnt[u]), int(ex[u]))) if kind == "ascending" else (lambda u: (-int(cnt[u]), int(ex[u])))
        misses = sorted((u for u in range(len(ex)) if not res[u]), key=key)
        g = p["gpu_base_us"] + (0 if kind == "no_hit" else p["gpu_hit_us"] * nres)
        if nres == 0 and kind != "base_always":
            g = 0.0
        c = p["cpu_base_us"] if (cpu_ok and misses and kind != "late_base") else 0.0
        ncpu = 0
        for u in misses:
            home = p["home_single"] and ntok > 1 and cnt[u] == 1
            gc = p["gpu_home_us"] if home else p["gpu_admit_us"]
            base = p["cpu_base_us"] if (kind == "base_each" or (kind == "late_base" and ncpu == 0)) else 0.0
            cc = base + p["cpu_expert_us"] + p["cpu_token_us"] * (int(cnt[u]) - 1)
            better = (max(c + cc, g) < max(c, g + gc)) if kind == "strict" else (max(c + cc, g) <= max(c, g + gc))
            if cpu_ok and ncpu < p["max_cpu"] and better:
                lanes[u], c, ncpu = 3, c + cc, ncpu + 1
            else:
                lanes[u] = 2 if home else 1
                g += gc
        return lanes
    return plan


@pytest.mark.parametrize("kind", ["strict", "ascending", "base_each", "no_hit", "late_base", "base_always"])
def test_planted_mistakes_fail_a_known_answer(kind):
    assert any(run_case(mutated(kind), c) != c[-1] for c in CASES), kind
    assert all(run_case(mutated("none"), c) == c[-1] for c in CASES)


def test_planned_step_admits_only_admit_lanes(oracle):
    """Two free slots, misses 0 (admit), 1 (home), 2 (CPU), 3 (admit): experts 0 and 3 take the slots; every miss
    counts; fresh marks the admitted ones."""
    t = oracle.SlotTable(1, 6, 2)
    el = oracle.expert_lanes(6, [0, 1, 2, 3], [oracle.LANE_ADMIT, oracle.LANE_HOME, oracle.LANE_CPU, oracle.LANE_ADMIT])
    jobs, ev = t.step(0, np.array([3, 1, 0, 2, 0], np.int64), 0, True, 8, elane=el)
    assert jobs.tolist() == [[0, 0], [3, 1]] and ev.tolist() == [-1, -1]
    assert t.stats[1] == 4 and t.stats[2] == 2 and t.fresh.tolist() == [1, 0, 0, 1, 0, 0]
    assert t.slotof[:6].tolist() == [0, -1, -1, 1, -1, -1]
    # next step: 0 and 3 hit; 1 still misses and is admitted now (no free slot: both pinned this step -> none)
    el = oracle.expert_lanes(6, [0, 1, 3], [oracle.LANE_VRAM, oracle.LANE_ADMIT, oracle.LANE_VRAM])
    jobs, _ = t.step(0, np.array([0, 1, 3], np.int64), 0, True, 8, elane=el)
    assert len(jobs) == 0 and t.stats[0] == 2 and t.stats[3] == 1


def test_request_and_selection(oracle):
    t = oracle.SlotTable(2, 8, 3)
    t.step(1, np.array([12, 14], np.int64), 10)               # experts 2, 4 of layer 1 resident
    ex, res, cnt = t.request(1, np.array([14, 9, 12, 12, 17, 18, 11], np.int64), 10)
    assert ex.tolist() == [1, 2, 4, 7] and res.tolist() == [0, 1, 1, 0] and cnt.tolist() == [1, 2, 1, 1]
    el = oracle.expert_lanes(8, ex, [oracle.LANE_CPU, oracle.LANE_VRAM, oracle.LANE_VRAM, oracle.LANE_HOME])
    sel = np.array([14, 9, 12, 12, 17, 18, 11], np.int64)
    w = np.array([0.5, 0.25, 1, 2, 0.125, 3, 4], np.float16)
    sg, wg, ln = oracle.planned_selection(sel, w, 10, el)
    assert sg.tolist() == [14, 9, 12, 12, 17, 18, -1]
    assert wg.tolist() == [0.5, 0.25, 1, 2, 0.125, 3, 0]
    assert ln.tolist() == [0, -1, 0, 0, 2, -1, 3]
