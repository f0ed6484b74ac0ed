"""Synthetic inputs for the five benchmark configurations.

Every random number comes from the project's own SplitMix64 streams (the
same generator as crates/llm-core/src/rng.rs:16-22), so a (config, data seed)
pair names one exact set of logits, histories and per-row RNG seeds. Inputs
are produced on the host with numpy and handed to both the GPU library and
the CPU oracle as the same bytes.

Configurations (B rows, V vocab, H history):
  1  B=1,    V=8192,   N(0, 2^2);                   T .8  k 40 p .95 min_p .05 rp 1.1  H 256 uniform
  2  B=64,   V=8192,   N(0, 3^2) + 12 at one spot;  T 1   k 50 p .9  min_p .1  rp 1.2  H 512 Zipf(1.1)
  3  B=256,  V=32000,  even rows N(0,.5^2), odd N(0,4^2); T .7 k 64 p .95 min_p .05 rp 1.15 H 1024 uniform
  4  B=1024, V=50257 (ld 50260), N(0, 1);           T 1   k 0  p .98 min_p 0   rp 1.0 (no history)
  5  B=512,  V=131072, Gumbel(0,1) + 0.02*i/(V-1);  T .9  k 0  p 1.0 min_p .02 rp 1.3  H 2048 Zipf(1.0)

Zipf histories draw a rank r in 1..V with P(r) ~ r^-s by inverse CDF and map
it to an id through a seeded permutation of the vocabulary. Config 5's
"0.02 * rank-linear trend" is read as a tilt linear in the id, i/(V-1).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
DEFAULT_DATA_SEED = 0x5C41F7A1D0C0FFEE
EOS_ID = 258

PARAMS_DTYPE = np.dtype(
    [
        ("temperature", "<f4"),
        ("top_k", "<u4"),
        ("top_p", "<f4"),
        ("min_p", "<f4"),
        ("repetition_penalty", "<f4"),
    ]
)


def splitmix64_outputs(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start..start+n-1 of a SplitMix64 generator seeded with `seed`.

    Output i (0-based) is mix(seed + (i+1) * 0x9E3779B97F4A7C15), which is what
    i+1 calls of rng.rs `next_u64` return.
    """
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * GOLDEN
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _substream(seed: int, tag: int) -> int:
    return int(splitmix64_outputs(seed ^ (tag * 0xD1B54A32D192ED03 & 0xFFFFFFFFFFFFFFFF), 1)[0])


def uniform01(seed: int, n: int) -> np.ndarray:
    """n doubles uniform in (0, 1) (53-bit, offset by half an ulp)."""
    z = splitmix64_outputs(seed, n)
    return ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)


def normal(seed: int, n: int) -> np.ndarray:
    """n standard normals by Box-Muller (float64)."""
    m = (n + 1) // 2
    u = uniform01(seed, 2 * m)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * m)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return out[:n]


def gumbel(seed: int, n: int) -> np.ndarray:
    return -np.log(-np.log(uniform01(seed, n)))


def zipf_ids(seed: int, n: int, V: int, s: float, perm: np.ndarray) -> np.ndarray:
    ranks = np.arange(1, V + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** (-s))
    cdf /= cdf[-1]
    r = np.searchsorted(cdf, uniform01(seed, n), side="left")
    r = np.minimum(r, V - 1)
    return perm[r].astype(np.uint32)


def permutation(seed: int, V: int) -> np.ndarray:
    return np.argsort(splitmix64_outputs(seed, V), kind="stable").astype(np.uint32)


@dataclass
class Workload:
    name: str
    B: int
    V: int
    ld: int
    logits: np.ndarray          # float32 [B, ld]
    params: np.ndarray          # PARAMS_DTYPE [1] (shared by all rows)
    hist: np.ndarray | None     # uint32 [sum H]
    hist_offsets: np.ndarray | None  # uint32 [B+1]
    rng_seeds: np.ndarray       # uint64 [B]
    H: int
    data_seed: int
    description: str = ""
    extra: dict = field(default_factory=dict)

    def bytes_per_row(self) -> int:
        """Algorithmic HBM bytes per row: logits + history (when the penalty
        is on) + RNG state in and out + the id out."""
        rp = float(self.params["repetition_penalty"][0])
        hist_bytes = 4 * self.H if (rp != 1.0 and self.H > 0) else 0
        return 4 * self.V + hist_bytes + 8 + 8 + 4


CONFIGS = {
    1: dict(B=1, V=8192, ld=8192, T=0.8, k=40, p=0.95, mp=0.05, rp=1.1, H=256, hist="uniform"),
    2: dict(B=64, V=8192, ld=8192, T=1.0, k=50, p=0.9, mp=0.1, rp=1.2, H=512, hist="zipf", s=1.1),
    3: dict(B=256, V=32000, ld=32000, T=0.7, k=64, p=0.95, mp=0.05, rp=1.15, H=1024, hist="uniform"),
    4: dict(B=1024, V=50257, ld=50260, T=1.0, k=0, p=0.98, mp=0.0, rp=1.0, H=0, hist=None),
    5: dict(B=512, V=131072, ld=131072, T=0.9, k=0, p=1.0, mp=0.02, rp=1.3, H=2048, hist="zipf", s=1.0),
}


def make_params(T: float, k: int, p: float, mp: float, rp: float) -> np.ndarray:
    prm = np.zeros(1, dtype=PARAMS_DTYPE)
    prm["temperature"] = T
    prm["top_k"] = k
    prm["top_p"] = p
    prm["min_p"] = mp
    prm["repetition_penalty"] = rp
    return prm


def _row_logits(cfg: int, b: int, V: int, seed: int) -> np.ndarray:
    rs = _substream(seed, 1000003 * (b + 1) + cfg)
    if cfg == 1:
        x = 2.0 * normal(rs, V)
    elif cfg == 2:
        x = 3.0 * normal(rs, V)
        spot = int(splitmix64_outputs(_substream(rs, 7), 1)[0] % np.uint64(V))
        x[spot] += 12.0
    elif cfg == 3:
        x = (0.5 if b % 2 == 0 else 4.0) * normal(rs, V)
    elif cfg == 4:
        x = normal(rs, V)
    elif cfg == 5:
        x = gumbel(rs, V) + 0.02 * (np.arange(V, dtype=np.float64) / (V - 1))
    else:
        raise ValueError(cfg)
    return x.astype(np.float32)


def make_workload(cfg: int, data_seed: int = DEFAULT_DATA_SEED, B: int | None = None,
                  V: int | None = None) -> Workload:
    """Build config `cfg` (1..5). B and V may be overridden (smaller parity
    cases of the same distribution); ld follows V (config 4 keeps the 16-byte
    padded stride)."""
    c = dict(CONFIGS[cfg])
    if B is not None:
        c["B"] = B
    if V is not None:
        c["V"] = V
        c["ld"] = V if cfg != 4 else (V + 3) // 4 * 4
    B_, V_, ld = c["B"], c["V"], c["ld"]
    logits = np.zeros((B_, ld), dtype=np.float32)
    for b in range(B_):
        logits[b, :V_] = _row_logits(cfg, b, V_, data_seed)
    H = c["H"]
    hist = offs = None
    if H and c["hist"]:
        if c["hist"] == "uniform":
            z = splitmix64_outputs(_substream(data_seed, 2), B_ * H)
            hist = (z % np.uint64(V_)).astype(np.uint32)
        else:
            perm = permutation(_substream(data_seed, 3), V_)
            hist = zipf_ids(_substream(data_seed, 4), B_ * H, V_, c["s"], perm)
        offs = (np.arange(B_ + 1, dtype=np.uint64) * H).astype(np.uint32)
    seeds = splitmix64_outputs(_substream(data_seed, 5), B_)
    return Workload(
        name=f"config{cfg}", B=B_, V=V_, ld=ld, logits=logits,
        params=make_params(c["T"], c["k"], c["p"], c["mp"], c["rp"]),
        hist=hist, hist_offsets=offs, rng_seeds=seeds, H=H if hist is not None else 0,
        data_seed=data_seed,
        description=f"B={B_} V={V_} T={c['T']} top_k={c['k']} top_p={c['p']} min_p={c['mp']} "
                    f"rep={c['rp']} H={H}",
    )
