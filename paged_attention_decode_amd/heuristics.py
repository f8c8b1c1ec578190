"""Split-count heuristic, mirrored in Python.

The launch uses the C++ implementation (``plan_impl`` in csrc/pa_decode.hip,
exposed as ``pad_decode_plan``); this module restates it so the choice can be
inspected and unit-tested on a host without a GPU, and the tests check that
both agree.  It replaces the reference's constant default
``_DEFAULT_NUM_SPLITS = 64`` (src/kernel_cuda_v4.py:16), which over-splits
large batches (profiles/notes.md:875-883 of the reference).

Inputs are shapes only (no ``seq_lens`` read, so no device sync):
batch, kv heads, head_dim, page_size, ``max_pages = block_table.shape[1]``
and the CU count.  Fitted to measured split-count sweeps of configurations
C2 (batch 1-64), C3 and C4 on MI355X: a power-of-two split count (or the
largest count that fits the workgroup budget, where that is 1.5 times as
many or more) with at least 16 blocks of 16 tokens per split; bandwidth-bound shapes get one
4-wave workgroup per CU, latency-bound ones (at most 16 blocks of work per
CU) 8-wave workgroups on at most half the CUs.  Bandwidth-bound shapes with
more than one (sequence, kv head) unit per two CUs and batch <= 256 get a grid of
OVERSUBSCRIBE_SPLITS items per unit (more below two units per CU, so that
the grid holds OVERSUBSCRIBE_GROUPS_PER_CU workgroups per CU), which the
kernel fills from the lengths: the static splits of the power-of-two rule
when every sequence is full, equal page chunks otherwise.  The same holds
from more than one unit per four CUs, where two static splits per unit
would leave CUs idle.
"""

from __future__ import annotations

from dataclasses import dataclass

BLOCK_TOKENS = 16          # tokens per wave iteration (one MFMA tile)
MAX_WAVES = 8              # waves per phase-1 workgroup (4 once the CUs are filled)
MAX_SPLITS = 1024          # PAD_MAX_SPLITS
MIN_BLOCKS = 16            # 16-token blocks per split, at least
MIN_BLOCKS_SHORT = 4       # the same for short latency-bound sequences (<= 16 splits)
LDS_BUDGET = 136 * 1024    # LDS of one workgroup: wave merge + MFMA staging
OVERSUBSCRIBE_SPLITS = 4   # items per unit on an oversubscribed grid, at least,
OVERSUBSCRIBE_GROUPS_PER_CU = 8  # and at least this many workgroups per CU
PLAN_MAX_BATCH = 256       # largest batch the in-kernel planner handles
TWO_LEVEL_SPLITS = 48      # units with more splits merge in two levels (groups of 16)


@dataclass(frozen=True)
class Plan:
    num_splits: int
    pages_per_split: int
    waves_per_group: int
    single_pass: bool
    workspace_bytes: int
    counters: int


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


def group_lds_bytes(nw: int, gqa: int, head_dim: int, engine: int = 0) -> int:
    """Dynamic LDS of a workgroup: per wave (m, l) [16] and O [gqa][D + 4] in fp32, plus for the MFMA
    engine a padded 16-row K staging tile per wave and, at head_dim 256, one padded 16-row Q^T copy."""
    stage = 16 * (2 * head_dim + 16) if engine == 0 else 0
    q_stage = stage if engine == 0 and head_dim >= 256 else 0
    return nw * (16 * 8 + gqa * (head_dim + 4) * 4 + stage) + q_stage


def pages_per_seq(batch: int, max_pages: int, csr: bool) -> int:
    """Pages of one sequence the plan assumes: the dense row width, or for a CSR index (max_pages = entries of
    ``indices``) the mean per sequence."""
    if max_pages <= 0:
        return 1
    if not csr or batch <= 1:
        return max_pages
    return _cdiv(max_pages, batch)


def plan(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, page_size: int, max_pages: int,
         num_splits: int = 0, num_cus: int = 256, engine: int = 0, csr: bool = False, kv_bytes: int = 2) -> Plan:
    """Same result as ``pad_decode_plan`` (``pad_decode_plan_csr`` with ``csr``) for valid arguments.

    ``kv_bytes=1`` gives the plan of an fp8-cache launch (pad_decode_launch_kv8): the same splits and
    scratch except where the fp16 plan is an oversubscribed grid (fp8 takes the 4-item grid from one
    unit per CU up only: never more scratch), 8-wave workgroups for its 128-byte rows at head_dim 128."""
    if num_cus <= 0:
        num_cus = 256
    gqa = num_q_heads // num_kv_heads
    mp = pages_per_seq(batch, max_pages, csr)
    units = max(batch, 1) * num_kv_heads
    blocks_per_seq = _cdiv(mp * page_size, BLOCK_TOKENS)
    latency_bound = units * blocks_per_seq <= 16 * num_cus
    if num_splits > 0:
        s = num_splits
        pps = _cdiv(mp, s)
    else:
        max_groups = num_cus // 2 if latency_bound else num_cus
        want = 1
        while want * 2 * units <= max_groups:
            want *= 2
        fit = max_groups // units
        if 2 * fit >= 3 * want:  # the largest count that fits, where it is 1.5x the power of two or more
            want = fit
        if oversubscribed(batch, num_kv_heads, max_pages, latency_bound, num_cus, kv_bytes):
            if kv_bytes == 1:  # fp8 caches: the 4-item grid from one unit per CU up
                want = OVERSUBSCRIBE_SPLITS
            else:
                want = max(OVERSUBSCRIBE_SPLITS, _cdiv(OVERSUBSCRIBE_GROUPS_PER_CU * num_cus, units))
                if head_dim * kv_bytes <= 128 and units <= num_cus:  # 8-wave workgroups: half the items
                    want //= 2
        cap = blocks_per_seq // MIN_BLOCKS
        if latency_bound:  # short sequences: down to 4 blocks per split, at most 16 splits
            cap = max(cap, min(blocks_per_seq // MIN_BLOCKS_SHORT, 16))
        cap = max(cap, 1)
        want = max(min(want, cap, MAX_SPLITS), 1)
        if csr:  # never more splits (scratch) than the dense plan of the same dims
            want = min(want, plan(batch, num_q_heads, num_kv_heads, head_dim, page_size, max_pages, 0, num_cus,
                                  engine).num_splits)
        pps = _cdiv(mp, want)
        s = _cdiv(mp, pps)
    nw = _cdiv(pps * page_size, BLOCK_TOKENS)
    narrow_rows = head_dim * kv_bytes <= 128 and units <= num_cus
    nw = min(nw, MAX_WAVES if latency_bound or narrow_rows else MAX_WAVES // 2)
    fixed = group_lds_bytes(0, gqa, head_dim, engine)
    per_wave = group_lds_bytes(1, gqa, head_dim, engine) - fixed
    # head_dim 256: at most 4 waves, one per SIMD, so a wave has the whole register file
    cap_w = max(min((LDS_BUDGET - fixed) // per_wave, 4 if head_dim >= 256 else MAX_WAVES), 1)
    nw = max(min(nw, cap_w), 1)
    single = s == 1
    ws = 0 if single else workspace_bytes(batch, num_kv_heads, gqa, head_dim, s)
    units = batch * num_kv_heads
    counters = 0 if single else units + (units * s if units * s > TWO_LEVEL_SPLITS else 0)
    return Plan(s, pps, nw, single, ws, counters)


def oversubscribed(batch: int, num_kv_heads: int, max_pages: int, latency_bound: bool, num_cus: int,
                   kv_bytes: int = 2) -> bool:
    """Heuristic shape planned in-kernel over an oversubscribed grid: more than one unit per two CUs,
    or more than one per four CUs where two static splits per unit leave CUs idle (fp8 caches: one
    unit per CU or more)."""
    units = max(batch, 1) * num_kv_heads
    if kv_bytes == 1:
        many = units >= num_cus
    else:
        many = units * 2 > num_cus or (units * 4 > num_cus and units * 2 < num_cus)
    return not latency_bound and many and batch <= PLAN_MAX_BATCH and max_pages < (1 << 23)


def workspace_bytes(batch: int, num_kv_heads: int, gqa: int, head_dim: int, num_splits: int) -> int:
    """256 B alignment slack + fp32 O [B, Hkv, S, gqa, D] + (m, l) [B, Hkv, S, gqa]."""
    rows = batch * num_kv_heads * num_splits * gqa
    return 256 + rows * head_dim * 4 + rows * 8
