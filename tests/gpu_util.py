"""Helpers shared by the GPU parity tests (inputs from the seeded device generator, the
same bytes copied to the host for the oracle)."""
import sys

import numpy as np

H, I, E = 2048, 512, 256


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def normwise_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def elementwise_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    floor = 1e-3 * np.sqrt((ref ** 2).mean())
    return float((np.abs(got - ref) / np.maximum(np.abs(ref), floor)).max())


class Layer:
    """One generated layer, resident on the GPU, with a lazily copied host view."""

    def __init__(self, pkg, orc, seed, hidden=H, inter=I, n_experts=E, dev=None):
        """The layer of generator stream `seed`, or the packed device buffer `dev`."""
        import torch
        self.pkg, self.orc = pkg, orc
        self.H, self.I, self.E = hidden, inter, n_experts
        self.dev = dev if dev is not None else pkg.gen_layer(hidden, inter, n_experts, seed)
        torch.cuda.synchronize()
        self._host = None

    def host(self):
        if self._host is None:
            self._host = self.orc.PackedLayer(self.dev.cpu().numpy(), self.H, self.I, self.E)
        return self._host


def sync():
    import torch
    torch.cuda.synchronize()
