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


def qwen3_config(shape="tiny", layers=2, vocab=1000):
    """Random-init Qwen3 configs: 'tiny' (hidden 512, 4 q / 2 kv heads) or
    'qwen3_4b' (hidden 2560, 32 q / 8 kv heads, intermediate 9728); head_dim
    128, RoPE theta 1e6, RMSNorm eps 1e-6 as in Qwen3-4B."""
    from transformers import Qwen3Config
    if shape == "qwen3_4b":
        dims = dict(hidden_size=2560, intermediate_size=9728, num_attention_heads=32, num_key_value_heads=8)
    else:
        dims = dict(hidden_size=512, intermediate_size=1024, num_attention_heads=4, num_key_value_heads=2)
    return Qwen3Config(vocab_size=vocab, num_hidden_layers=layers, head_dim=128, rope_theta=1e6,
                       rms_norm_eps=1e-6, max_position_embeddings=8192, tie_word_embeddings=False,
                       attention_dropout=0.0, **dims)


def make_qwen3(shape="tiny", layers=2, seed=0):
    import torch
    from transformers import Qwen3ForCausalLM
    torch.manual_seed(seed)
    cfg = qwen3_config(shape, layers)
    cfg._attn_implementation = "eager"
    m = Qwen3ForCausalLM(cfg).float()
    m.train()
    return m
