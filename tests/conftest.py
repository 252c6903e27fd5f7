import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libg3attn.so on the GPU)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def pytest_runtest_setup(item):
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] start {item.nodeid}", flush=True)
