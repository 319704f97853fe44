"""geometric-nn-ops-torch, MI355X-native: the inference forward of the triangle ops runs on
hand-written gfx950 HIP kernels behind a C ABI (``libgnn_hip.so``); backward passes,
CPU tensors and shapes the kernels do not cover run a pure-torch differentiable path.

Kernels are namespaced by family as submodules:

* ``geometric_nn_ops_torch.triangle`` -- protein-folding (triangle) ops.
"""

__version__ = "0.1.0"
