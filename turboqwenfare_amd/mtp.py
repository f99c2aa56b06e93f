"""MTP verification accounting (host side).

Mirrors ``src/runtime/mtp.rs`` of the reference: ``expert_bytes`` (:38-42),
``MtpStatistics`` (:48-83), ``verify_pair`` (:98-104), ``MtpController``
(:112-168) and ``union_bandwidth`` (:185-203), plus the k-draft
generalisations the HIP verify step needs (the union of M = k+1 routes in
first-demand order, experts/mod.rs:268-275, and the expected tokens per
verify step).  This is integer/host logic; the device computes the same union
inside its route kernel.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Sequence

HIDDEN = 2048
EXPERT_WIDTH = 512
TOP_K = 8
Q4K_BLOCK_BYTES = 144
Q4_0_BLOCK_BYTES = 18


def _q4k_bytes(rows: int, cols: int) -> int:
    return rows * (cols // 256) * Q4K_BLOCK_BYTES


def _q4_0_bytes(rows: int, cols: int) -> int:
    return rows * (cols // 32) * Q4_0_BLOCK_BYTES


def expert_bytes() -> int:
    """mtp.rs:38-42: one routed expert's Q4_K gate + up + down bytes."""
    return (_q4k_bytes(EXPERT_WIDTH, HIDDEN) + _q4k_bytes(EXPERT_WIDTH, HIDDEN)
            + _q4k_bytes(HIDDEN, EXPERT_WIDTH))


def expert_bytes_q4_0() -> int:
    """The same for the Q4_0 group-32 layout (equal: both are 4.5 bits/weight)."""
    return (_q4_0_bytes(EXPERT_WIDTH, HIDDEN) * 2 + _q4_0_bytes(HIDDEN, EXPERT_WIDTH))


@dataclass
class MtpStatistics:
    """mtp.rs:48-83."""

    drafted_tokens: int = 0
    accepted_tokens: int = 0
    target_backbone_passes: int = 0
    emitted_tokens: int = 0

    def acceptance_rate(self) -> float:
        return 0.0 if self.drafted_tokens == 0 else self.accepted_tokens / self.drafted_tokens

    def emitted_tokens_per_target_pass(self) -> float:
        if self.target_backbone_passes == 0:
            return 0.0
        return self.emitted_tokens / self.target_backbone_passes

    def record(self, accepted: bool, emitted: int, target_passes: int) -> None:
        self.drafted_tokens += 1
        if accepted:
            self.accepted_tokens += 1
        self.target_backbone_passes += target_passes
        self.emitted_tokens += emitted

    def record_verify(self, k: int, accepted: int) -> None:
        """One k-draft verify pass: each draft is recorded as accepted or not
        (drafts after the first rejection count as drafted, not accepted) and
        accepted + 1 tokens are emitted for one target pass."""
        for i in range(k):
            self.drafted_tokens += 1
            if i < accepted:
                self.accepted_tokens += 1
        self.target_backbone_passes += 1
        self.emitted_tokens += accepted + 1


@dataclass(frozen=True)
class VerifyOutcome:
    """mtp.rs:90-96: Accepted{emitted_tokens} / Rejected{emitted_tokens}."""

    accepted: bool
    emitted_tokens: int


def verify_pair(target_prediction_after_boundary: int, draft_token: int) -> VerifyOutcome:
    """mtp.rs:98-104: greedy k = 1 verification."""
    if target_prediction_after_boundary == draft_token:
        return VerifyOutcome(True, 2)
    return VerifyOutcome(False, 1)


@dataclass
class MtpController:
    """mtp.rs:112-168: rolling-window hysteresis (+0.10 enable, -0.05 disable)."""

    window_capacity: int
    window: list = field(default_factory=list)
    enabled: bool = False
    enable_threshold: float = 0.10
    disable_threshold: float = -0.05

    def rolling_net_benefit(self) -> float:
        return 0.0 if not self.window else sum(self.window) / len(self.window)

    def record_and_decide(self, emitted_tokens: int) -> bool:
        net = float(emitted_tokens) - 1.0
        if len(self.window) == self.window_capacity:
            self.window.pop(0)
        self.window.append(net)
        if len(self.window) < self.window_capacity:
            return self.enabled
        rolling = self.rolling_net_benefit()
        if not self.enabled and rolling > self.enable_threshold:
            self.enabled = True
        elif self.enabled and rolling < self.disable_threshold:
            self.enabled = False
        return self.enabled


@dataclass(frozen=True)
class UnionBandwidth:
    """mtp.rs:177-183."""

    union_experts: int
    union_bytes: int
    separate_experts_sum: int
    separate_bytes_sum: int
    saved_bytes: int


def union_bandwidth(boundary: Sequence[int], draft: Sequence[int]) -> UnionBandwidth:
    """mtp.rs:185-203."""
    return routes_union_bandwidth([boundary, draft])


def routes_union(routes: Sequence[Sequence[int]]) -> list[int]:
    """Distinct experts of M routes in first-demand order (experts/mod.rs:268-275)."""
    union: list[int] = []
    for route in routes:
        for e in route:
            if e not in union:
                union.append(int(e))
    return union


def routes_union_bandwidth(routes: Sequence[Sequence[int]],
                           per_expert: int | None = None) -> UnionBandwidth:
    """union_bandwidth generalised to the M = k+1 routes of one verify pass."""
    per = expert_bytes() if per_expert is None else per_expert
    union = routes_union(routes)
    separate = sum(len(r) for r in routes)
    ub, sb = len(union) * per, separate * per
    return UnionBandwidth(len(union), ub, separate, sb, max(sb - ub, 0))


def expected_tokens_per_step(alpha: float, k: int) -> float:
    """E[emitted tokens per verify step] with per-draft acceptance alpha:
    (1 - alpha^(k+1)) / (1 - alpha) (Leviathan et al. 2023, eq. 1)."""
    if alpha >= 1.0:
        return float(k + 1)
    return (1.0 - alpha ** (k + 1)) / (1.0 - alpha)
