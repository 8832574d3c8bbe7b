"""CPU oracle of the mHC path: test infrastructure, never product code.

``reference`` restates the math in PyTorch (float64-capable, autograd);
``csk`` loads the C restatement of Sinkhorn-Knopp and its explicit adjoint
(built by ``oracle/Makefile`` into ``oracle/_build``).
"""
