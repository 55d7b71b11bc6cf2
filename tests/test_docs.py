"""Every PJRTX_* environment switch the plugin, its Python bindings or
bench.py reads is listed in INTEGRATION.md's switch table (no GPU)."""
import pathlib
import re

ROOT = pathlib.Path(__file__).resolve().parent.parent


def test_every_environment_switch_is_documented():
    files = list((ROOT / "pjrtx_amd" / "csrc").rglob("*.cc")) + list((ROOT / "pjrtx_amd" / "csrc").rglob("*.h")) + \
        list((ROOT / "pjrtx_amd" / "csrc").rglob("*.hip")) + list((ROOT / "pjrtx_amd").glob("*.py")) + [ROOT / "bench.py"]
    used = set()
    for f in files:
        used |= set(re.findall(r'"(PJRTX_[A-Z0-9_]+)"', f.read_text()))
    doc = (ROOT / "INTEGRATION.md").read_text()
    missing = sorted(e for e in used if e not in doc)
    assert used and not missing, f"undocumented switches: {missing}"
