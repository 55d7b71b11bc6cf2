import os
import pathlib
import subprocess
import sys
import textwrap

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (runs on the MI355X box)")


@pytest.fixture(scope="session")
def plugin():
    from pjrtx_amd.pjrt import plugin as get
    return get()


@pytest.fixture(scope="session")
def client(plugin):
    from pjrtx_amd.pjrt import Client
    if plugin.device_count() == 0:
        pytest.fail("GPU test ran on a host without a visible HIP device")
    c = Client()
    yield c


_RUN_ONE = textwrap.dedent("""
    import sys, numpy as np
    sys.path.insert(0, sys.argv[1])
    from pjrtx_amd.pjrt import Client
    d = np.load(sys.argv[2])
    exe = Client().compile(open(sys.argv[3]).read())
    dts = [None if t == "" else str(t) for t in d["dtypes"]]
    outs = exe(*[d[f"a{i}"] for i in range(int(d["n"]))], dtypes=dts)
    np.savez(sys.argv[4], *outs)
""")


@pytest.fixture
def run_fresh(tmp_path):
    """Compiles and runs a program in a new process with extra environment
    (for settings read once per process, such as the XCD placement probe);
    returns its outputs."""
    def run(text, args, dtypes, env):
        (tmp_path / "p.mlir").write_text(text)
        np = __import__("numpy")
        np.savez(tmp_path / "in.npz", n=len(args), dtypes=np.array(["" if t is None else t for t in dtypes]),
                 **{f"a{i}": a for i, a in enumerate(args)})
        r = subprocess.run([sys.executable, "-c", _RUN_ONE, str(ROOT), str(tmp_path / "in.npz"),
                            str(tmp_path / "p.mlir"), str(tmp_path / "out.npz")],
                           env=dict(os.environ, **env), capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        z = np.load(tmp_path / "out.npz")
        return [z[f"arr_{i}"] for i in range(len(z.files))]
    return run
