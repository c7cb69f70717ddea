"""Shared setup for the parity tests: seeded Maple-shaped layers for both the HIP path and the oracle."""
import numpy as np

import maplemoe as M
import pyoracle as O

SEED = 20261201


def relmax(a, b):
    """max |a - b| / max |b| (max-normalised relative difference, the tolerance metric of the north star)"""
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    den = np.abs(b).max()
    return float(np.abs(a - b).max() / (den if den > 0 else 1.0))


def normed_hidden(seed, sid, nb):
    """N(0,1) hidden states, RMS-normed with unit weight (the configs' MoE input), through the oracle's rmsnorm"""
    x = M.synth_hidden(seed, sid, nb)
    hn = np.empty_like(x)
    for b in range(nb):
        O.oracle().mo_rmsnorm(O._p(x[b]), None, M.H, O._p(hn[b]))
    return x, hn


class HostLayer:
    """One synthetic layer on the host: expert block, router, oracle expert table."""

    def __init__(self, seed, L, dist=0):
        self.L = L
        self.blk = M.synth_layer_block(seed, L)
        self.router = M.synth_router(seed, L, dist)
        self.table = O.experts_table(self.blk)
