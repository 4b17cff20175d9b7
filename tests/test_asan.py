"""The C oracle and the product's host training code under AddressSanitizer
and UBSan (CPU only): oracle/asan/asan_driver.cpp exercises both on small
inputs and edge cases; any out-of-bounds access, leak or undefined behaviour
aborts the run.  The driver also checks the host training code bit for bit
against the oracle (rotation, 1-D k-means, Lloyd-Max codebooks)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_oracle_and_host_train_under_asan(tmp_path):
    exe = str(tmp_path / "asan_driver")
    src = [os.path.join(ROOT, "oracle", "asan", "asan_driver.cpp"),
           os.path.join(ROOT, "jhq_gpu_amd", "csrc", "host_train.cpp")]
    flags = ["-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
             "-ffp-contract=off", "-pthread"]
    obj = str(tmp_path / "jhq_oracle.o")
    r = subprocess.run(["gcc", "-std=gnu11", "-mfma", "-c", os.path.join(ROOT, "oracle",
                        "jhq_oracle.c"), "-o", obj] + flags, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run(["g++", "-std=c++17", "-mfma"] + flags + src + [obj, "-o", exe, "-lm"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0 and "asan driver ok" in r.stdout, (r.stdout[-2000:], r.stderr[-4000:])
