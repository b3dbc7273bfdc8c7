"""CPU oracle of the reference operators.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg import this package, and only to check or time
against it. The ``laplacianformer_amd`` product path never imports it.
"""
from .ref import *  # noqa: F401,F403
