"""Deterministic synthetic workloads for the five benchmark configurations.

Generator (identical wherever it runs, numpy only): counter-based splitmix64
(``x -> mix(seed + (stream << 40) + counter)``), uniforms from the top 53 bits,
normals by Box--Muller.  Seed ``0x5EED0000 + config_id``.

* neighbour vector: direction = normalise(3 normals); radius ``R u^(1/3)``,
  rejected (redrawn with fresh counters) while below ``r_min``;
* neighbour id ``j = (i + 1 + floor(u (N-1))) mod N`` (uniform over ``j != i``);
* species uniform in ``[0, S)``; node features and radial-mix weights normal;
* CSR by centre: ``row_offsets[i] = i K``, edges of a row in draw order, which
  is the stable ``(center, draw)`` order of ``prepare_carrier_scatter_segments``
  (reference ``ye3t/runtime/execution_plan.py:9316-9434``).

ChebExpCos cutoff = ball radius; ``lambda = 0.5723`` (the reference's own radial
fixture value, ``tests/cpp/test_runtime_core_standalone.cpp:611``).
"""

from dataclasses import dataclass, field

import numpy as np

from ye3t_amd.ace.plan import ACEFeatureSpec

LAMBDA = 0.5723
_MASK = (1 << 64) - 1


def _splitmix(x):
    x = (x + np.uint64(0x9E3779B97F4A7C15)) & np.uint64(_MASK)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


class CounterRNG:
    def __init__(self, seed):
        self.seed = np.uint64(seed)

    def bits(self, stream, counter):
        counter = np.asarray(counter, dtype=np.uint64)
        with np.errstate(over="ignore"):
            return _splitmix(self.seed + (np.uint64(stream) << np.uint64(40)) + counter)

    def uniform(self, stream, counter):
        return (self.bits(stream, counter) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)

    def normal(self, stream, count, offset=0):
        """Box--Muller normals from pairs of uniforms of one stream."""
        half = (count + 1) // 2
        idx = np.arange(half, dtype=np.uint64) * np.uint64(2) + np.uint64(2 * offset)
        u1 = self.uniform(stream, idx)
        u2 = self.uniform(stream, idx + np.uint64(1))
        u1 = np.where(u1 <= 0.0, 2.0 ** -53, u1)
        rad = np.sqrt(-2.0 * np.log(u1))
        z = np.empty(2 * half)
        z[0::2] = rad * np.cos(2.0 * np.pi * u2)
        z[1::2] = rad * np.sin(2.0 * np.pi * u2)
        return z[:count]


def neighbor_vectors(rng, count, radius, r_min):
    """``count`` vectors uniform in the shell ``r_min <= r <= radius``."""
    out = np.empty((count, 3))
    todo = np.arange(count)
    round_ = 0
    while todo.size:
        base = round_ * count
        d = rng.normal(1, 3 * todo.size, offset=3 * base).reshape(-1, 3)
        n = np.linalg.norm(d, axis=1)
        n = np.where(n == 0.0, 1.0, n)
        u = rng.uniform(2, np.uint64(base) + todo.astype(np.uint64))
        r = radius * np.cbrt(u)
        ok = r >= r_min
        out[todo[ok]] = d[ok] / n[ok, None] * r[ok, None]
        todo = todo[~ok]
        round_ += 1
    return out


@dataclass
class DensityWorkload:
    atom_count: int
    neighbors_per_atom: int
    radius: float
    r_min: float
    n_max: int
    l_max: int
    species_count: int = 0          # one-hot species channels when > 0
    node_channels: int = 0          # node-feature channels (channel-wise products) when > 0
    config_id: int = 0
    extra: dict = field(default_factory=dict)

    @property
    def channel_count(self):
        return self.species_count or self.node_channels or 1

    @property
    def radial_rows(self):
        return 1 if self.node_channels else self.n_max + 1

    def generate(self):
        rng = CounterRNG(0x5EED0000 + self.config_id)
        N, K = self.atom_count, self.neighbors_per_atom
        E = N * K
        centers = np.repeat(np.arange(N, dtype=np.int64), K)
        u = rng.uniform(3, np.arange(E, dtype=np.uint64))
        neighbors = (centers + 1 + np.floor(u * (N - 1)).astype(np.int64)) % N
        vectors = neighbor_vectors(rng, E, self.radius, self.r_min)
        out = {
            "atom_count": N, "edge_count": E, "centers": centers,
            "row_offsets": np.arange(N + 1, dtype=np.int64) * K, "neighbors": neighbors,
            "edge_vectors": vectors, "channel_count": self.channel_count, "n_max": self.n_max,
            "l_max": self.l_max, "cutoff": float(self.radius), "lambda": LAMBDA, "epsilon": 1e-12,
            "species": None, "node_features": None, "radial_mix": None,
        }
        if self.species_count:
            s = rng.uniform(4, np.arange(N, dtype=np.uint64))
            out["species"] = np.minimum(np.floor(s * self.species_count), self.species_count - 1).astype(np.int32)
        if self.node_channels:
            C = self.node_channels
            out["node_features"] = rng.normal(5, N * C).reshape(N, C)
            out["radial_mix"] = rng.normal(6, C * (self.n_max + 1)).reshape(C, self.n_max + 1) / np.sqrt(self.n_max + 1)
        return out


@dataclass
class Config:
    config_id: int
    name: str
    density: DensityWorkload = None
    feature_spec: ACEFeatureSpec = None
    dtypes: tuple = ("f64",)
    channelwise: bool = False       # samples are (atom, channel) rows of A
    accumulate: str = None          # type of the arithmetic (None: the storage dtype)
    density_dtype: str = None       # storage type of A (None: the arithmetic type)
    note: str = ""

    def samples(self):
        d = self.density
        return d.atom_count * (d.node_channels if self.channelwise else 1)


def config(config_id, *, atom_count=None):
    """Configuration ``config_id`` (1..5); ``atom_count`` shrinks it for parity tests."""
    if config_id == 1:
        return Config(1, "readme-quickstart-sector", dtypes=("f64",),
                      note="content (1,1,2), input_Ls (1,1,0); factors [4096, 8, 3] and [4096, 8, 1]")
    if config_id == 2:
        d = DensityWorkload(atom_count or 10000, 24, 5.0, 0.8, 8, 3, config_id=2)
        spec = ACEFeatureSpec(channel_count=9, l_max=3, nu_max=3, targets=(0,), parity="even")
        return Config(2, "scalar-ace-single-species", d, spec, ("f64",))
    if config_id == 3:
        d = DensityWorkload(atom_count or 20000, 32, 5.0, 0.8, 10, 4, species_count=4, config_id=3)
        spec = ACEFeatureSpec(channel_count=44, l_max=4, nu_max=4, targets=(0,), parity="even",
                              radial_per_species=11, caps={1: (11, 0), 2: (11, 4), 3: (4, 3), 4: (2, 2)})
        return Config(3, "scalar-ace-4-species", d, spec, ("f64", "f32"))
    if config_id == 4:
        d = DensityWorkload(atom_count or 50000, 24, 5.0, 0.8, 8, 3, node_channels=16, config_id=4)
        spec = ACEFeatureSpec(channel_count=1, l_max=3, nu_max=3, nu_min=3, targets=(0, 1, 2))
        # fp32 storage, fp64 arithmetic: over the full 800 000 samples a density
        # accumulated in fp32 leaves 4.8e-5 column error in B, while an fp64
        # accumulation rounded once to an fp32 density leaves 1.3e-5 (fp64 A: 5e-6)
        return Config(4, "equivariant-message-couplings", d, spec, ("f32",), channelwise=True,
                      accumulate="f64", density_dtype="f32")
    if config_id == 5:
        d = DensityWorkload(atom_count or 200000, 48, 5.5, 0.8, 12, 6, species_count=8, config_id=5)
        spec = ACEFeatureSpec(channel_count=104, l_max=6, nu_max=4, targets=(0, 1, 2), parity="any",
                              radial_per_species=13, caps={1: (13, 2), 2: (4, 6), 3: (1, 3), 4: (1, 1)})
        # fp32 storage, fp64 intermediates: odd-L couplings of two l=6 densities of
        # neighbouring radial channels cancel to ~1e-4 of their terms, beyond what
        # fp32 intermediates resolve at the 2e-5 feature tolerance
        return Config(5, "large-scale-stress", d, spec, ("f32",), accumulate="f64")
    raise ValueError(f"unknown config {config_id}")


def config1_factors(batch=4096, channels=8):
    """Config 1 supplied factors: ``A_{1,1}[B, C, 3]`` and ``A_{2,0}[B, C, 1]``, N(0,1)."""
    rng = CounterRNG(0x5EED0000 + 1)
    a11 = rng.normal(1, batch * channels * 3).reshape(batch, channels, 3)
    a20 = rng.normal(2, batch * channels).reshape(batch, channels, 1)
    return a11, a20
