"""Conversion of the reference's per-head weight tensors to the dense C x C
matrices that ``slime_ca_set_params`` takes.

The reference keeps its projection weights per head (``MultiHeadCAState``,
slime/core/pseudopod.cu:29-38; allocated at slime/runtime.cu:77-82):

    perception_weights   [NUM_HEADS][CHANNELS][HIDDEN_DIM]
    interaction_weights  [NUM_HEADS][CHANNELS][HIDDEN_DIM]
    value_weights        [NUM_HEADS][HIDDEN_DIM][CHANNELS]

and its kernel (multi_head_ca_kernel, pseudopod.cu:79-119) uses, for head h, only
the D x D block at the top left of each slab (D = HEAD_DIM = 64):

    perception[i]  = ReLU(sum_{c < D} x_h[c] * perception_weights[h][c][i])
    interaction[i] = GELU_tanh(sum_{j < D} perception[j] * interaction_weights[h][j][i])
    output[i]      = sum_{j < HIDDEN_DIM} interaction[j % D] * value_weights[h][j][i]

(the perception there also sums the 3 x 3 neighbourhood before the product; the
step built here projects the cell itself). Those per-head products are the
block-diagonal case of the dense projections: block (h, h) of W_P and W_I is the
head's D x D block, and block (h, h) of W_V is the value block folded over the
HIDDEN_DIM / D repeats that ``j % D`` reads,

    W_V[hD + j][hD + i] = sum_r value_weights[h][j + r D][i],

every other block zero. With ``pvi_chain = 1`` (I from P, V from I) the step then
computes the reference's chain; with ``pvi_chain = 0`` it computes all three from
the state with the same blocks. The flow kernels [H][3][3] flatten to K [H][9]
(tap 3 (dy + 1) + (dx + 1)) and head_mixing_weights [H][H] is M as it stands.
"""
from __future__ import annotations

import numpy as np


def from_reference_weights(perception: np.ndarray, interaction: np.ndarray, value: np.ndarray,
                           head_mixing: np.ndarray, flow_kernels: np.ndarray,
                           head_dim: int = 64) -> dict:
    """Dense ``slime_ca_params`` arrays (one pod) from the reference's tensors.

    perception, interaction: [H][CHANNELS][HIDDEN]; value: [H][HIDDEN][CHANNELS];
    head_mixing: [H][H]; flow_kernels: [H][3][3]. Returns WP, WI, WV [1][C][C],
    K [1][H][9], M [1][H][H] as fp32 with C = H * head_dim (mu and sigma are not
    part of the reference's state and come from the caller).
    """
    perception = np.asarray(perception, dtype=np.float32)
    interaction = np.asarray(interaction, dtype=np.float32)
    value = np.asarray(value, dtype=np.float32)
    H = perception.shape[0]
    D = int(head_dim)
    hidden = value.shape[1]
    if perception.shape[1] < D or perception.shape[2] < D or interaction.shape[1] < D \
            or interaction.shape[2] < D or value.shape[2] < D or hidden < D:
        raise ValueError("every per-head slab must hold at least a head_dim x head_dim block")
    if interaction.shape[0] != H or value.shape[0] != H:
        raise ValueError("perception, interaction and value must have the same number of heads")
    C = H * D
    WP = np.zeros((C, C), np.float32)
    WI = np.zeros((C, C), np.float32)
    WV = np.zeros((C, C), np.float32)
    for h in range(H):
        blk = slice(h * D, (h + 1) * D)
        WP[blk, blk] = perception[h, :D, :D]
        WI[blk, blk] = interaction[h, :D, :D]
        # output[i] reads interaction[j % D] for every j < HIDDEN: the rows of the
        # value slab that share j % D add up (in fp64, then rounded once).
        fold = np.zeros((D, D), np.float64)
        for j in range(hidden):
            fold[j % D] += value[h, j, :D]
        WV[blk, blk] = fold.astype(np.float32)
    K = np.asarray(flow_kernels, dtype=np.float32).reshape(H, 9)
    M = np.asarray(head_mixing, dtype=np.float32).reshape(H, H)
    return {"WP": WP[None], "WI": WI[None], "WV": WV[None], "K": K[None].copy(),
            "M": M[None].copy()}
