"""Algorithmic work and traffic of the attention path (the roofline's numerators).

Units of work: one visible (query, key) pair of one (batch, head).
  N_vis per (b, h): S^2 non-causal, S(S+1)/2 causal, W*S - W(W-1)/2 for a
  causal window W < S; with s sinks the span W - s takes that form and the
  sinks add sum_i min(s, max(0, i - (W - s) + 1)).
FLOPs credited (2 flop per multiply-add, softmax/exp not counted, recompute
not credited):
  forward            4*D per pair   (S = Q K^T, O = P V)
  backward          10*D per pair   (S, dP, dV, dQ, dK)
  fwd + bwd         14*D per pair   <- the headline metric
Per launch of each kernel, counting every product that kernel performs:
  attn_fwd           4*D per pair
  attn_bwd_dkdv      8*D per pair   (S, dP, dV, dK)
  attn_bwd_dq        6*D per pair   (S, dP, dQ)
Compulsory HBM bytes (T = B*S*H*D*elem, L = B*H*S*4):
  fwd+bwd  12*T + 4*L ; attn_bwd_delta reads O, dO and writes Delta: 2*T + L.
"""

from __future__ import annotations

# MI355X published peaks (dense, no sparsity).
PEAK_TFLOPS = {"bf16": 2516.6, "f16": 2516.6, "f32": 157.3}
PEAK_HBM_GBS = 8000.0


def nvis(S: int, causal: bool = True, window: int = 0, sinks: int = 0, block: int = 0) -> int:
    if not causal:
        return S * S
    if block and block > 1:                 # query i sees keys [0, min(S, (i // block + 1) * block))
        return sum(min(block, S - b0) * min(S, b0 + block) for b0 in range(0, S, block))
    span = window - sinks if window and window > 0 else 0
    if 0 < span < S:
        n = S - span                  # queries that see sinks beyond their span
        extra = (n * (n + 1) // 2 if n <= sinks
                 else sinks * (sinks + 1) // 2 + sinks * (n - sinks))
        return span * S - span * (span - 1) // 2 + extra
    return S * (S + 1) // 2


def flops(B: int, H: int, S: int, D: int, causal: bool = True, window: int = 0,
          bwd: bool = True, sinks: int = 0, block: int = 0) -> float:
    """Headline algorithmic FLOPs: 4*B*H*D*N_vis forward (+ 10*B*H*D*N_vis backward)."""
    return (14.0 if bwd else 4.0) * B * H * D * nvis(S, causal, window, sinks, block)


KERNEL_FLOPS_PER_PAIR_D = {"attn_fwd": 4, "attn_bwd_dkdv": 8, "attn_bwd_dq": 6,
                           "attn_bwd_dq+delta": 6}


def kernel_flops(kernel: str, B: int, H: int, S: int, D: int, causal: bool = True,
                 window: int = 0, sinks: int = 0, block: int = 0) -> float:
    return KERNEL_FLOPS_PER_PAIR_D[kernel] * B * H * D * float(nvis(S, causal, window, sinks,
                                                                     block))


def tensor_bytes(B: int, S: int, H: int, D: int, elem: int) -> int:
    return B * S * H * D * elem


def delta_bytes(B: int, S: int, H: int, D: int, elem: int) -> int:
    return 2 * tensor_bytes(B, S, H, D, elem) + 4 * B * H * S


def compulsory_bytes(B: int, S: int, H: int, D: int, elem: int) -> int:
    return 12 * tensor_bytes(B, S, H, D, elem) + 4 * 4 * B * H * S
