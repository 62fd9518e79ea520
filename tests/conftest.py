import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT / "tests", ROOT / "web-engine_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C-ABI library")


import pytest  # noqa: E402


@pytest.fixture(scope="session")
def graph():
    """One context on cuda:0 for the GPU tests (fails loudly when libwe.so or the GPU is missing)."""
    import we
    g = we.Graph(0)
    info = g.device_info()
    print(f"\n[gpu] {info}", flush=True)
    assert info["arch"].startswith("gfx950"), info
    yield g
    g.destroy()


@pytest.fixture
def tune(graph):
    """Pins kernel choices of the session's context for one test (graph.set_tuning: tune(gemm_cfg=0, ...)); the
    previous values come back when the test ends."""
    saved = {}

    def set_(**switches):
        for key, value in switches.items():
            prev = graph.set_tuning(key, value)
            saved.setdefault(key, prev)

    yield set_
    for key, value in saved.items():
        graph.set_tuning(key, value)


@pytest.fixture(autouse=True)
def _announce(request):
    """Names each GPU test before it runs, so a run that dies still shows which case it was on."""
    if request.node.get_closest_marker("gpu"):
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
