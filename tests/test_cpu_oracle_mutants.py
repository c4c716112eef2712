"""The oracle's sampler and collect pins (test_cpu_sampling.py) reject the
plausible slips they are meant to catch: each mutant below is a copy of
oracle/oracle.cpp with one such slip, compiled into a temporary directory and
loaded in place of the oracle (MG_ORACLE_LIB), and each must fail at least one
pin. The unmutated source, compiled the same way, must pass them all. CPU only;
nothing here touches the product."""
import concurrent.futures as cf
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "oracle.cpp")
PINS = os.path.join(ROOT, "tests", "test_cpu_sampling.py")

COLLECT_LOOP = ("for (uint32_t t = 0; t < horizon; ++t) {  // model/ppo.h:727-733\n"
                "                size_t k = (size_t)t * n + i;\n")

# name: (text in oracle.cpp, replacement) -- each text occurs exactly once
MUTANTS = {
    "categorical_le": ("if (u < acc) {", "if (u <= acc) {"),
    "box_muller_u1_is_u": ("float u1 = 1.0f - (float)(xs_next(rng) >> 8)", "float u1 = 0.0f + (float)(xs_next(rng) >> 8)"),
    "box_muller_odd_takes_cos": ("float zk = (k & 1u) ? z1 : z0;", "float zk = z0;"),
    "box_muller_sin_cos_swapped": ("float zk = (k & 1u) ? z1 : z0;", "float zk = (k & 1u) ? z0 : z1;"),
    "collect_reset_before_sample": (COLLECT_LOOP,
                                    COLLECT_LOOP + "                if (done[i]) { env_reset(env, s, rng[i]); done[i] = 0; }\n"),
    "collect_no_first_step": ("if (first) {  // model/ppo.h:720-722", "if (first && false) {  // model/ppo.h:720-722"),
    "collect_no_obs_copy": ("std::memcpy(obs_slots + (size_t)i * O, obs_slots + ((size_t)horizon * n + i) * O, O * 4);",
                            "(void)0;"),
    "collect_bootstrap_on_last_step": ("forward_row(net, obs_slots + ((size_t)horizon * n + i) * O, head_out",
                                       "forward_row(net, obs_slots + ((size_t)(horizon - 1) * n + i) * O, head_out"),
}


def compile_copy(tmp, name, text):
    cpp = os.path.join(tmp, f"{name}.cpp")
    with open(cpp, "w") as f:
        f.write(text)
    so = os.path.join(tmp, f"lib{name}.so")
    # the oracle's own flags (oracle/Makefile) at -O1 for a faster build; without
    # fast-math and with contraction off, the IEEE arithmetic is the same at any -O
    cmd = ["g++", "-O1", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-shared",
           "-I", os.path.join(ROOT, "oracle"), cpp, "-o", so, "-lpthread"]
    subprocess.run(cmd, check=True, capture_output=True)
    return so


def run_pins(so):
    env = dict(os.environ, MG_ORACLE_LIB=so)
    r = subprocess.run([sys.executable, "-m", "pytest", PINS, "-x", "-q", "-p", "no:cacheprovider"], cwd=ROOT,
                       env=env, capture_output=True, text=True, timeout=600)
    return r.returncode, r.stdout[-2000:]


@pytest.fixture(scope="module")
def builds(tmp_path_factory):
    tmp = str(tmp_path_factory.mktemp("oracle_mutants"))
    with open(SRC) as f:
        src = f.read()
    texts = {"original": src.replace('#include "../include/mg/math.h"',
                                     f'#include "{os.path.join(ROOT, "include", "mg", "math.h")}"')}
    for name, (old, new) in MUTANTS.items():
        assert src.count(old) == 1, f"mutant {name}: anchor text must occur once in oracle.cpp"
        texts[name] = texts["original"].replace(old, new)
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        futs = {name: ex.submit(compile_copy, tmp, name, text) for name, text in texts.items()}
        sos = {name: f.result() for name, f in futs.items()}
    with cf.ThreadPoolExecutor(max_workers=4) as ex:
        futs = {name: ex.submit(run_pins, so) for name, so in sos.items()}
        return {name: f.result() for name, f in futs.items()}


def test_unmutated_copy_passes_the_pins(builds):
    rc, out = builds["original"]
    assert rc == 0, out


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_mutant_fails_a_pin(builds, name):
    rc, out = builds[name]
    assert rc == 1, f"mutant {name} was not caught (pytest exit {rc}):\n{out}"
