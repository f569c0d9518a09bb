import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); skipped when none is visible")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


class Node:
    """Minimal duck-typed tree node for the oracle (token_ids, children)."""

    def __init__(self, token_ids, name=""):
        self.token_ids = list(token_ids)
        self.children = []
        self.name = name

    def add_child(self, token_ids, name=""):
        c = Node(token_ids, name)
        self.children.append(c)
        return c

    @property
    def is_leaf(self):
        return not self.children


def load_golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def forest_from_spec(spec_nodes, node_cls=Node, token_base=1):
    """Build a forest from [{'name','len','parent'}] in DFS pre-order."""
    objs = []
    roots = []
    tok = token_base
    for nd in spec_nodes:
        ids = list(range(tok, tok + nd["len"]))
        tok += nd["len"]
        if nd["parent"] < 0:
            n = node_cls(ids)
            roots.append(n)
        else:
            n = objs[nd["parent"]].add_child(ids)
        try:
            n.name = nd["name"]
        except AttributeError:
            pass
        objs.append(n)
    return roots, objs


@pytest.fixture
def c1_spec():
    return load_golden("c1_tree.json")


@pytest.fixture
def q1_spec():
    return load_golden("q1_chain.json")
