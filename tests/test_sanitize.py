"""The host C code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

tests/sanitize/host_checks.c links the real host layer (attn_flash.c, attn_synth.c) and the real
oracle (oracle/attn_oracle.c) with stand-in launchers that write every scratch slot the kernels
could write into a host scratch of exactly attn_flash_scratch_bytes(D, bk). A wrong carve or a
split count past the slot capacity is a heap overflow; bad size arithmetic is UB. No GPU."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")


def test_host_code_under_asan_ubsan():
    r = subprocess.run(["make", "-B", "-s", "-C", SAN], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([os.path.join(SAN, "host_checks")], capture_output=True, text=True,
                       timeout=300, env=env)
    print(r.stdout[-3000:], r.stderr[-3000:])
    assert r.returncode == 0
    assert "HOST_CHECKS OK" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr
