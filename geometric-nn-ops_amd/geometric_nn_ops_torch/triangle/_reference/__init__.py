"""Pure-torch, autograd-differentiable forms of the triangle ops.

This is the product's fallback for what the HIP kernels do not serve: calls that need a
backward, CPU tensors, dtypes without a kernel and shapes outside the kernels' limits
(the reference routes the same cases to its own torch path, triangle/_trimul.py:31-36).
The test oracle is a separate CPU restatement under the repository's oracle/ directory.
"""
