"""The integration boundary as the repository's integration guide states it:
the ctypes binding block the guide shows runs unchanged against the built
library, and ``import sparselab`` resolves to this package after
``install_as_sparselab()``.

CPU: the block's struct matches the library's ``slk_csr`` mirror field for
field, and the alias serves the reference's module names. GPU: the block's
``spmm_simd`` gives ``sparsecore_amd.spmm``'s bits, and a SparseLinear built
through ``sparselab.nn`` trains.
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


def _binding_block() -> str:
    text = (REPO / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    found = [b for b in blocks if "class slk_csr" in b]
    assert len(found) == 1, "the integration guide must hold exactly one binding block"
    return found[0]


def _run_block() -> dict:
    from sparsecore_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libsparsecore_amd.so is not built")
    os.environ["SLK_LIBRARY"] = str(_lib.LIB_PATH)
    ns: dict = {}
    exec(compile(_binding_block(), "integration-guide", "exec"), ns)
    return ns


def test_binding_block_matches_the_library_struct():
    from sparsecore_amd import _lib

    ns = _run_block()
    mine, ref = ns["slk_csr"], _lib.CsrView
    assert [f for f, _ in mine._fields_] == [f for f, _ in ref._fields_]
    assert [t for _, t in mine._fields_] == [t for _, t in ref._fields_]
    assert ctypes.sizeof(mine) == ctypes.sizeof(ref)
    assert ns["_lib"].slk_abi_version() == _lib.ABI_VERSION


def test_sparselab_alias_serves_the_reference_names():
    # a fresh interpreter: the alias edits sys.modules
    code = (
        "import sparsecore_amd as s\n"
        "s.install_as_sparselab()\n"
        "import sparselab, sparselab.ops, sparselab.nn, sparselab.layout, sparselab.router\n"
        "from sparselab import PaddedCSR, spmm, SparseLinear, SparsityAlgorithm, Static, "
        "DynamicSparsityAlgorithm, SET, RigL\n"
        "from sparselab.layout import transpose_with_perm, from_dense\n"
        "from sparselab.ops import _cached_transpose\n"
        "assert sparselab is s and sparselab.nn is s.nn and sparselab.ops is s.ops\n"
        "s.install_as_sparselab()  # idempotent\n"
        "import types, sys\n"
        "sys.modules['sparselab'] = types.ModuleType('sparselab')\n"
        "try:\n"
        "    s.install_as_sparselab()\n"
        "except RuntimeError as e:\n"
        "    assert 'already imported' in str(e)\n"
        "else:\n"
        "    raise SystemExit('a foreign sparselab was shadowed')\n"
        "s.install_as_sparselab(force=True)\n"
        "assert sys.modules['sparselab'] is s\n"
        "print('ok')\n")
    env = dict(os.environ, PYTHONPATH=str(REPO) + os.pathsep + os.environ.get("PYTHONPATH", ""))
    out = subprocess.run([sys.executable, "-c", code], cwd=REPO, env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0 and out.stdout.strip().endswith("ok"), out.stderr[-2000:]


@pytest.mark.gpu
def test_binding_block_spmm_matches_the_package(dev):
    import torch

    import sparsecore_amd
    from sparsecore_amd import PaddedCSR

    ns = _run_block()
    g = torch.Generator().manual_seed(7)
    dense = torch.randn(300, 500, generator=g) * (torch.rand(300, 500, generator=g) < 0.1)
    W = PaddedCSR.from_dense(dense, padding_ratio=0.2).to(dev)
    X = torch.randn(500, 1024, generator=g).to(dev)
    got = ns["spmm_simd"](W, X)
    want = sparsecore_amd.spmm(W, X)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.gpu
def test_sparselinear_trains_through_the_sparselab_name(dev):
    import torch

    import sparsecore_amd

    saved = {k: v for k, v in sys.modules.items() if k == "sparselab" or k.startswith("sparselab.")}
    try:
        sparsecore_amd.install_as_sparselab(force=True)
        import sparselab
        from sparselab.nn import SparseLinear

        torch.manual_seed(0)
        layer = SparseLinear(96, 80, sparsity=0.8).to(dev)
        algo = sparselab.SET(sparsity=0.8, drop_fraction=0.3, update_freq=1, seed=0)
        layer.apply(algo)  # the reference's attach idiom (sparselab/router.py:121)
        opt = torch.optim.SGD(layer.parameters(), lr=0.1)
        x = torch.randn(64, 96, device=dev)
        target = torch.randn(64, 80, device=dev)
        losses = []
        for _ in range(5):
            opt.zero_grad()
            loss = ((layer(x) - target) ** 2).mean()
            loss.backward()
            opt.step()
            algo.step()
            losses.append(loss.item())
        assert all(v == v for v in losses) and losses[-1] < losses[0]
        assert layer._csr.topology_version > 0
    finally:
        for k in [k for k in sys.modules if k == "sparselab" or k.startswith("sparselab.")]:
            del sys.modules[k]
        sys.modules.update(saved)
