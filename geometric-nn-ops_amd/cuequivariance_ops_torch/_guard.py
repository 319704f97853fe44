"""Import-time checks of the shim (reference hipequivariance_ops_torch/
cuequivariance_ops_torch/_guard.py:1-63): a real cuequivariance ops wheel claiming the same
module name is an error (which one Python imports would be arbitrary); a
cuequivariance-torch frontend other than the one this API follows is a warning."""

import warnings
from importlib import metadata

CONFLICTING_DISTRIBUTIONS = ("cuequivariance-ops-torch", "cuequivariance-ops-torch-cu12",
                             "cuequivariance-ops-torch-cu13")
FRONTEND = "cuequivariance-torch"
FRONTEND_VERSION = "0.9.1"


def installed() -> set[str]:
    return {(d.metadata["Name"] or "").lower() for d in metadata.distributions()} - {""}


def check() -> None:
    names = installed()
    clash = sorted(set(CONFLICTING_DISTRIBUTIONS) & names)
    if clash:
        raise RuntimeError(
            "cuequivariance_ops_torch shim: the NVIDIA ops wheel(s) " + ", ".join(clash)
            + " provide the same module; uninstall them (pip uninstall " + " ".join(clash)
            + ") to run on the HIP kernels")
    try:
        version = metadata.version(FRONTEND)
    except metadata.PackageNotFoundError:
        return
    if version != FRONTEND_VERSION:
        warnings.warn(f"cuequivariance_ops_torch shim: written against {FRONTEND}=={FRONTEND_VERSION}, "
                      f"found {version}; the API may differ", RuntimeWarning, stacklevel=2)
