"""Build flags: every HIP source is compiled without packed-fp32 instructions,
and the sanitizer build (swiftllm_amd/sanitize.py) applies each -fsanitize=
to the host pass only, never to device code. (Imports are inside the tests:
the sanitizer build script is not shipped to GPU boxes, where these CPU tests
are collected but not run.)"""


def test_packed_fp32_disabled_for_every_hip_compile():
    from swiftllm_amd import build

    flags = build.FLAGS
    i = flags.index("-packed-fp32-ops")
    assert flags[i - 3:i + 1] == ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def test_sanitizers_apply_to_the_host_pass_only():
    from swiftllm_amd import sanitize

    flags = sanitize.HOST_SANITIZE
    for i, f in enumerate(flags):
        if f.startswith("-fsanitize") or f.startswith("-fno-sanitize"):
            assert i > 0 and flags[i - 1] == "-Xarch_host", f
