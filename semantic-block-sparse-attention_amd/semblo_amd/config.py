"""Paper defaults and the cluster-count rule of the flat partition.

Values follow semblo/vllm_plugin/paper_defaults.py:42-104 (PAPER_ENV,
PAPER_TEXT_CONFIG, budget K = capacity / 16) and state.py:586-597 (the
power-of-two cluster count).
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field

PAGE = 16                    # SEMBLO_FA3_BODY / SEMBLO_FA3_ALIGN
FLAT_UNIT_TOKENS = 2048      # SEMBLO_FLAT_UNIT_TOKENS
FLAT_MIN_CLUSTERS_LOG2 = 7   # SEMBLO_FLAT_MIN_CLUSTERS_LOG2
BUDGET_DIVISOR = 16          # K = L / 16
CAPACITY_MULTIPLE = 16384


def flat_cluster_count(length: int, target_size: int, *, min_clusters: int = 64,
                       max_clusters: int = 16384) -> int:
    """flat_index.py:81-84."""
    return int(min(max(length // max(target_size, 1), min_clusters), max_clusters, length))


def fitted_sink_tokens() -> int:
    """SEMBLO_SINK_TOKENS (default 0, off): with S > 0 the fitted partition reserves
    cluster 0 for positions 0..S-1, its descriptor zero, and every selection takes it
    first inside a budget reduced by S (state.py:21-23, fused_prefill.py:192-216)."""
    return max(0, int(os.environ.get("SEMBLO_SINK_TOKENS", "0") or "0"))


def check_sink_partition(sink: int, length: int, fit_length: int, num_clusters: int) -> None:
    """The settings a reserved sink cluster does not compose with (state.py:26-34, the
    checks that apply to this build's partition)."""
    if sink % 16:
        raise RuntimeError(f"SEMBLO_SINK_TOKENS={sink}: a multiple of 16 keeps the sink cluster page-aligned")
    if length <= sink or fit_length - sink < 2 * num_clusters:
        raise RuntimeError(f"SEMBLO_SINK_TOKENS={sink} leaves too few keys ({length:,} in the prompt, "
                           f"{fit_length:,} to fit) for {num_clusters - 1} clusters")


def default_suffix_reserve(room: int | None = None) -> int:
    """Generated positions a layer's decode state holds room for (arena.py:50-63):
    SEMBLO_SUFFIX_RESERVE if set, else the model's room for generated tokens capped at
    65,536, else 65,536."""
    env = os.environ.get("SEMBLO_SUFFIX_RESERVE")
    if env is not None:
        return int(env)
    if room is not None:
        return max(1, min(65536, int(room)))
    return 65536


def num_flat_clusters(length: int, unit_tokens: int = FLAT_UNIT_TOKENS,
                      min_log2: int = FLAT_MIN_CLUSTERS_LOG2) -> int:
    """state.py:586-597: a power of two, floored at 2^min_log2, capped by the prompt."""
    min_c_log2 = max(3, int(min_log2))
    raw = flat_cluster_count(length, unit_tokens)
    c = 1 << max(min_c_log2, (max(raw, 1) - 1).bit_length())
    return min(c, 1 << (int(length).bit_length() - 1))


@dataclass
class SembloRuntimeConfig:
    """The settings of one sparse layer on the paper path (config.py:93-198 subset)."""

    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    selection_temperature: float = 0.1      # paper (paper_defaults.py:89)
    bucket_size_penalty: float = 0.25       # paper (paper_defaults.py:82)
    query_chunk_size: int = 8192            # paper (paper_defaults.py:99)
    target_tokens: int = 0                  # 0: L / 16
    codebook_seed: int = 0
    layer_idx: int = 0
    flat_unit_tokens: int = FLAT_UNIT_TOKENS
    flat_min_clusters_log2: int = FLAT_MIN_CLUSTERS_LOG2
    page_align: int = PAGE
    kmeans_sample_size: int = 8192
    dense_prefix_x: int = 4                 # SEMBLO_FA3_DENSE_PREFIX_X
    iters: int = 16
    decode_num_splits: int = 56             # splits of the decode step (with the suffix splits:
                                            # 64 blocks per KV head)
    decode_suffix_splits: int = 8           # SEMBLO_DECODE_SUFFIX_SPLITS
    suffix_block: int = 256
    suffix_reserve: int = field(default_factory=lambda: default_suffix_reserve())
    sm_scale: float | None = None           # None: head_dim ** -0.5
    suffix_shuffle_seed: int | None = None  # suffix blocks in a shuffled physical order (a paged
                                            # cache's page order); None: in order
    decode_capacity: int = 0                # > 0: one decode arena for prompts up to this length,
                                            # made before any request and adopted into by each
                                            # (SEMBLO_FULL_GRAPH_DECODE, arena.py:66-253); the
                                            # decode budget is then budget(decode_capacity)
    # decode's own budget (SEMBLO_DECODE_TARGET_TOKENS, config.py:262-268 of the reference);
    # 0: decode selects on the prefill's budget.  The prompt length reads every cluster.
    decode_target_tokens: int = field(default_factory=lambda: int(
        os.environ.get("SEMBLO_DECODE_TARGET_TOKENS", "0") or 0))

    @property
    def scale(self) -> float:
        return self.sm_scale if self.sm_scale is not None else self.head_dim ** -0.5

    def budget(self, prompt_length: int) -> int:
        return int(self.target_tokens) if self.target_tokens > 0 else max(1, prompt_length // BUDGET_DIVISOR)
