"""The C++ mirror of the reference backend (include/vapi_kv.hpp), run by its
own test program tests/cpp/backend_tests.cpp: the reference's cache,
attention and block-method tests restated in C++ against libvapi_kv.so.
The host-only part runs here; the rest needs a GPU."""
import subprocess
import sys
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
BIN = HERE / "cpp" / "_build" / "backend_tests"


def _binary(build_if_missing: bool) -> Path:
    sys.path.insert(0, str(HERE / "cpp"))
    import build as cpp_build  # tests/cpp/build.py
    if not cpp_build.is_current():
        # A binary built against another version of the C header would hand
        # the library descriptors of another layout: never run one.
        if not build_if_missing:
            pytest.fail(f"{BIN} is missing or older than its sources "
                        "(python tests/cpp/build.py)")
        cpp_build.build()
    return BIN


def _run(args):
    res = subprocess.run([str(_binary(build_if_missing="--host-only" in args)), *args],
                         capture_output=True, text=True, timeout=300)
    print(res.stdout)
    print(res.stderr, file=sys.stderr)
    assert res.returncode == 0, res.stdout + res.stderr
    return res.stdout


def test_the_host_side_of_the_cpp_mirror():
    out = _run(["--host-only"])
    assert "validate_names_the_first_violation_as_the_reference_does ... ok" in out


@pytest.mark.gpu
def test_the_reference_backend_tests_pass_through_the_cpp_mirror():
    out = _run([])
    for name in ("a_write_spanning_non_adjacent_blocks_lands_in_exactly_those_slots",
                 "a_sliding_window_hides_keys_older_than_the_window",
                 "the_flash_kernel_matches_the_cpu_reference_in_bf16",
                 "copy_blocks_copies_every_layer_k_and_v"):
        assert f"{name} ... ok" in out
