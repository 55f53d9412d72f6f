"""End-to-end prefill through llama.cpp with this backend loaded as a ggml plugin: the
random-init Llama-3-8B Q4_K GGUF, 2048 prompt tokens, micro-batches of 512, the host's weight
repack off (ggml-rocket's README.md:82-95 and MODELS.md:65-74 protocol: `llama-bench -p 2048
-n 0 -b 512 -ub 512 -nr 1`), the backend's teardown lines (`[routes]`, `[f16-resident]` ...)
collected from the log, and the CPU backend alone on the same GGUF beside it.

    python ggml-rocket_amd/llama_bench.py --llama-cpp /path/to/llama.cpp [--gguf model.gguf]
                                          [--reps 3] [--dry-run]

It builds `lib/libggml-mi355x.so` against that checkout (`make -C ggml-rocket_amd ggml
HOST_GGML_DIR=...`) when the library is missing, writes the GGUF with llama3_gguf.py when the file
is missing, runs llama-bench with `GGML_BACKEND_PATH` pointing at the plugin and
`MI355X_QUANT_RESIDENT=1`, and prints one JSON line. Without a llama.cpp build (no
`build/bin/llama-bench`) it says so and exits with status 2; `--dry-run` prints the commands
without running anything.
"""
import argparse
import json
import os
import re
import shlex
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PLUGIN = os.path.join(HERE, "lib", "libggml-mi355x.so")


def bench_cmd(llama_bench: str, gguf: str, reps: int, repack: bool):
    return [llama_bench, "-m", gguf, "-p", "2048", "-n", "0", "-b", "512", "-ub", "512",
            "-nr", "0" if repack else "1", "-r", str(reps), "-o", "json"]


def parse_tps(stdout: str):
    """avg_ts of the prompt test in llama-bench's JSON output."""
    try:
        rows = json.loads(stdout)
    except json.JSONDecodeError:
        m = re.search(r"\[\s*\{.*\}\s*\]", stdout, re.S)
        if not m:
            return None
        rows = json.loads(m.group(0))
    for r in rows:
        if int(r.get("n_prompt", 0)) > 0 and int(r.get("n_gen", 0)) == 0:
            return float(r["avg_ts"])
    return None


def backend_lines(stderr: str):
    return [ln.strip() for ln in stderr.splitlines() if re.search(r"\[(routes|f16-resident|dq-cache|moe)\]", ln)]


def main():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--llama-cpp", required=True, help="a llama.cpp checkout with its build in build/bin")
    p.add_argument("--gguf", default=os.path.join(tempfile.gettempdir(), "llama3-8b-random-q4k.gguf"),
                   help="the model (written there by llama3_gguf.py when missing; about 4.9 GB)")
    p.add_argument("--reps", type=int, default=3)
    p.add_argument("--dry-run", action="store_true")
    a = p.parse_args()
    bin_dir = os.path.join(a.llama_cpp, "build", "bin")
    llama_bench = os.path.join(bin_dir, "llama-bench")
    make = ["make", "-C", HERE, "ggml", f"HOST_GGML_DIR={a.llama_cpp}", f"GGML_LIB_DIR={bin_dir}"]
    gen = [sys.executable, os.path.join(HERE, "llama3_gguf.py"), a.gguf]
    env_dev = {"GGML_BACKEND_PATH": PLUGIN, "MI355X_QUANT_RESIDENT": "1"}
    dev_cmd = bench_cmd(llama_bench, a.gguf, a.reps, repack=False)
    cpu_cmd = bench_cmd(llama_bench, a.gguf, 1, repack=True)
    if a.dry_run:
        print(json.dumps({"build": None if os.path.exists(PLUGIN) else shlex.join(make),
                          "gguf": None if os.path.exists(a.gguf) else shlex.join(gen),
                          "device": " ".join(f"{k}={v}" for k, v in env_dev.items()) + " " + shlex.join(dev_cmd),
                          "cpu": shlex.join(cpu_cmd)}))
        return 0
    if not os.path.exists(llama_bench):
        print(f"llama_bench.py: no llama-bench under {bin_dir}: build llama.cpp first "
              f"(cmake -B build && cmake --build build)", file=sys.stderr)
        return 2
    if not os.path.exists(PLUGIN):
        subprocess.run(make, check=True)
    if not os.path.exists(a.gguf):
        os.makedirs(os.path.dirname(os.path.abspath(a.gguf)), exist_ok=True)
        subprocess.run(gen, check=True)
    dev = subprocess.run(dev_cmd, env={**os.environ, **env_dev}, capture_output=True, text=True)
    cpu = subprocess.run(cpu_cmd, env={k: v for k, v in os.environ.items() if k != "GGML_BACKEND_PATH"},
                         capture_output=True, text=True)
    out = {"metric": "llama.cpp prefill tok/s (pp2048, -b 512 -ub 512, repack off), MI355X plugin",
           "value": parse_tps(dev.stdout), "unit": "tok/s", "cpu_backend_tok_s": parse_tps(cpu.stdout),
           "gguf": os.path.abspath(a.gguf), "plugin": PLUGIN, "reps": a.reps,
           "backend_log": backend_lines(dev.stderr), "status": [dev.returncode, cpu.returncode]}
    print(json.dumps(out))
    return 0 if dev.returncode == 0 else 1


if __name__ == "__main__":
    sys.exit(main())
