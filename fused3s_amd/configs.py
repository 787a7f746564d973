"""The five workloads of the path (synthetic, deterministic).

1-2: citation-style power-law graph of Cora's size (2,708 nodes, ~10,556
     directed edges + self-loops), d=64, H=1, Q/K/V ~ U[-1, 1].  Config 1 is
     the CPU reference run, config 2 the same inputs on the GPU.
3:   sparser Citeseer-sized graph (3,327 nodes, ~9,104 edges + self-loops,
     many degree-1 and isolated-before-self-loop nodes), U[-1, 1].
4:   1,000,000-node power-law graph, mean degree 16, exponent 2.2, random
     node order (tiles mostly 1-3 nnz), N(0, 1): the memory-bound gather
     regime the bench line is quoted on.
5:   2,400,000-node stochastic block model, 4,096-node communities, 80 %
     intra-community edges, mean degree ~50, community-ordered ids,
     H=4 heads x d=64, N(0, 1).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .graph import features_f16, powerlaw_graph, sbm_graph


@dataclass(frozen=True)
class Config:
    cfg: int
    name: str
    kind: str            # "powerlaw" | "sbm"
    n: int
    H: int
    normal: bool
    seed: int
    target_edges: int = 0
    gamma: float = 0.0
    max_degree: float = 0.0
    community: int = 0
    mean_degree: float = 0.0
    p_intra: float = 0.0
    d: int = 64

    def graph(self) -> tuple[np.ndarray, np.ndarray]:
        """(row_ptr, col_idx): symmetric, sorted unique columns, self-loops."""
        if self.kind == "powerlaw":
            return powerlaw_graph(self.n, self.target_edges, self.gamma, self.max_degree,
                                  permute=True, self_loops=True, seed=self.seed)
        return sbm_graph(self.n, self.community, self.mean_degree, self.p_intra,
                         self_loops=True, seed=self.seed)

    def features(self, tensor: int, rows: int | None = None) -> np.ndarray:
        """fp16 [n][H][d] values of Q (0), K (1) or V (2)."""
        rows = self.n if rows is None else rows
        f = features_f16(self.seed, tensor, rows * self.H * self.d, self.normal)
        return f.reshape(rows, self.H, self.d)


CONFIGS = {
    1: Config(1, "cora-like-cpu", "powerlaw", 2708, 1, False, 42, target_edges=10556,
              gamma=2.5, max_degree=170),
    2: Config(2, "cora-like-gpu", "powerlaw", 2708, 1, False, 42, target_edges=10556,
              gamma=2.5, max_degree=170),
    3: Config(3, "citeseer-like-sparse", "powerlaw", 3327, 1, False, 43, target_edges=9104,
              gamma=2.8, max_degree=99),
    4: Config(4, "powerlaw-1M", "powerlaw", 1_000_000, 1, True, 44, target_edges=16_000_000,
              gamma=2.2, max_degree=16384),
    5: Config(5, "sbm-2.4M-h4", "sbm", 2_400_000, 4, True, 45, community=4096,
              mean_degree=50.0, p_intra=0.8),
}
