"""Host-side checks of the benchmark contract and of where the oracle may be used.

* ``bench.py --gpus N`` with N > 1 exits with a message (one GPU only) before it
  touches a GPU.
* The oracle is test infrastructure: in ``bench.py`` only the ``cpu_baseline`` leg
  imports it, ``__graft_entry__`` only in ``smoke()``, and no module of the
  package imports it at all.  Checked on the syntax trees, so a stray import
  anywhere else (module level or another function) fails here.
"""
import ast
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _oracle_imports(path):
    """(enclosing function name or None, line) of every import of the oracle package."""
    tree = ast.parse(open(path).read(), filename=path)
    found = []

    def visit(node, func):
        for child in ast.iter_child_nodes(node):
            f = child.name if isinstance(child, (ast.FunctionDef, ast.AsyncFunctionDef)) else func
            if isinstance(child, ast.ImportFrom) and child.module and \
                    child.module.split(".")[0] == "oracle":
                found.append((func, child.lineno))
            elif isinstance(child, ast.Import) and any(
                    a.name.split(".")[0] == "oracle" for a in child.names):
                found.append((func, child.lineno))
            visit(child, f)

    visit(tree, None)
    return found


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2, (r.returncode, r.stdout, r.stderr)
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_oracle_only_in_bench_cpu_baseline():
    uses = _oracle_imports(os.path.join(ROOT, "bench.py"))
    assert uses, "the CPU baseline leg is expected to use the oracle"
    assert all(func == "cpu_baseline" for func, _ in uses), uses


def test_oracle_only_in_smoke():
    uses = _oracle_imports(os.path.join(ROOT, "__graft_entry__.py"))
    assert uses and all(func == "smoke" for func, _ in uses), uses


def test_package_never_imports_oracle():
    pkg = os.path.join(ROOT, "gpt_from_scratch_amd")
    offenders = []
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                p = os.path.join(dirpath, f)
                offenders += [(os.path.relpath(p, ROOT), line) for _, line in _oracle_imports(p)]
    assert offenders == []


def test_summarize_reads_rocprof_csv(tmp_path):
    """``bench.py --summarize DIR`` averages rocprofv3's per-dispatch CSV rows
    per kernel and grid: durations (end - start, ns -> µs), the back-to-back
    time of consecutive dispatches, scratch bytes and counter values."""
    d = tmp_path / "host" / "123"
    d.mkdir(parents=True)
    (d / "run_kernel_trace.csv").write_text(
        '"Kind","Kernel_Name","Start_Timestamp","End_Timestamp","Scratch_Size","Grid_Size_X"\n'
        '"KERNEL_DISPATCH","void mi::(anonymous namespace)::k_bwd<mi::BF16, 64>(mi::AttnArgs, int)",'
        '1000,56000,0,256\n'
        '"KERNEL_DISPATCH","void mi::(anonymous namespace)::k_bwd<mi::BF16, 64>(mi::AttnArgs, int)",'
        '60000,117000,0,256\n'
        '"KERNEL_DISPATCH","k_fwd",120000,141000,16,512\n')
    (d / "run_counter_collection.csv").write_text(
        '"Dispatch_Id","Grid_Size","Kernel_Name","Counter_Name","Counter_Value"\n'
        '1,256,"void mi::(anonymous namespace)::k_bwd<mi::BF16, 64>(mi::AttnArgs, int)",'
        '"FETCH_SIZE",100.0\n'
        '2,256,"void mi::(anonymous namespace)::k_bwd<mi::BF16, 64>(mi::AttnArgs, int)",'
        '"FETCH_SIZE",102.0\n')
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--summarize",
                        str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.splitlines()
    # back-to-back: (117000 - 1000) ns over 2 dispatches
    assert "| k_bwd<BF16, 64> [grid 256] | 2 | 56.000 | 55.000 | 57.000 | 58.000 | 0 |" in lines
    assert "| k_fwd [grid 512] | 1 | 21.000 | 21.000 | 21.000 | - | 16 |" in lines
    assert "| k_bwd<BF16, 64> [grid 256] | 2 | 101.0 | 100.0 | 102.0 |" in lines


def test_profiler_regions_are_harmless_without_a_profiler():
    """roctxProfilerResume / Pause without a profiler attached (or without the
    roctx library) do nothing and raise nothing."""
    from gpt_from_scratch_amd.profiler_regions import ProfilerRegions
    r = ProfilerRegions()
    r.resume()
    r.pause()
