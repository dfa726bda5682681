"""The resident store's eviction policy (strata-rs_amd/csrc/store.hpp), on the
CPU: least-recently-used first until the new tensor fits, a tensor larger
than the budget admitted alone into an empty store (as the reference's
WeightCache::insert, crates/strata-backend-wgpu/src/gpu.rs:88-112), and the
one addition here: entries pinned by the current call are never victims,
and when they keep the store over budget the admission is refused."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def policy(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:  # pragma: no cover - g++ is part of the image
        pytest.skip("no g++")
    exe = str(tmp_path_factory.mktemp("store") / "store_policy")
    subprocess.run([gxx, "-O1", "-std=c++17", "-Wall", "-Werror", "-fsanitize=address,undefined",
                    os.path.join(HERE, "store_policy.cpp"), "-o", exe], check=True)

    def run(*cases):
        text = "\n".join(cases) + "\n"
        out = subprocess.run([exe], input=text, capture_output=True, text=True, check=True).stdout
        return out.strip().split("\n")

    return run


def test_fits_without_eviction(policy):
    assert policy("100 10 5 1:40:1:1 2:40:2:2") == ["ok"]


def test_lru_order(policy):
    # 1 is least recently used, then 3, then 2
    assert policy("100 30 9 1:40:1:1 2:40:7:7 3:20:4:4") == ["ok 1"]
    assert policy("100 50 9 1:40:1:1 2:40:7:7 3:20:4:4") == ["ok 1 3"]
    assert policy("100 95 9 1:40:1:1 2:40:7:7 3:20:4:4") == ["ok 1 3 2"]


def test_reference_three_matrices_case(policy):
    # gpu.rs:577-599: 24 MiB budget, three 10 MiB matrices in turn: the third
    # evicts the first
    mib = 1 << 20
    assert policy(f"{24 * mib} {10 * mib} 3 1:{10 * mib}:1:1 2:{10 * mib}:2:2") == ["ok 1"]


def test_larger_than_budget_admitted_alone(policy):
    assert policy("100 150 9 1:40:1:1 2:40:2:2") == ["ok 1 2"]
    assert policy("100 150 9") == ["ok"]


def test_pinned_entries_are_never_victims(policy):
    # entry 1 is the oldest but pinned by call 9: 2 goes instead
    assert policy("100 50 9 1:40:1:9 2:40:7:7") == ["ok 2"]


def test_pinned_entries_that_cannot_make_room_refuse(policy):
    # the MoE case: gate and up pinned by this call, down does not fit beside them
    assert policy("100 60 9 1:40:5:9 2:40:6:9") == ["oom"]
    # a partial eviction is not enough either: nothing is evicted, refused
    assert policy("100 60 9 1:40:5:9 2:30:1:1 3:30:6:9") == ["oom"]


def test_pin_of_an_earlier_call_does_not_protect(policy):
    assert policy("100 60 10 1:40:5:9 2:40:6:9") == ["ok 1"]


def test_ties_in_the_clock_break_by_key(policy):
    assert policy("100 30 9 7:40:3:3 5:40:3:3") == ["ok 5"]


def test_the_moe_budget_two_of_three(policy):
    # the MoE config's expert tensors: gate and up 113,246,208 B (Q4_K), down
    # 165,150,720 B (Q6_K); a budget holding two of them but not three
    g, d = 128 * 2048 * 432, 128 * 768 * 1680
    budget = g + d
    # gate and up admitted in this call; down does not fit beside them
    assert policy(f"{budget} {d} 4 1:{g}:1:4 2:{g}:2:4") == ["oom"]
    # a later call admits down by evicting the least recently used of them
    assert policy(f"{budget} {d} 5 1:{g}:1:4 2:{g}:2:4") == ["ok 1"]
