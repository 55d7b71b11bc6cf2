"""Client-level PJRT families on the GPU: the topology description and its
serialized form (reference: src/plugin/topology.zig:85-108, 152-154: the same
fields in the same order)."""
import re

import pytest

pytestmark = pytest.mark.gpu


def test_topology_serializes_platform_and_every_device(client):
    s = client.topology_serialized()
    parts = s.split(";")
    assert parts[0] == "platform=" + client.platform_name
    assert re.fullmatch(r"version=.+", parts[1])
    n = int(parts[2].removeprefix("devices="))
    assert n == len(client.devices) >= 1
    devs = parts[3:]
    assert len(devs) == n
    for i, d in enumerate(devs):
        m = re.fullmatch(r"device=(\d+):(\d+):0:(.+)", d)
        assert m and int(m.group(1)) == i and int(m.group(2)) == i, d
    assert client.topology_serialized() == s  # stable; each copy freed by its deleter
