"""Expert-product oracle (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Dense per-token restatement of vLLM's fused_experts as the router-split
entry calls it (src/sluice/offloader.py:2590-2599): for every (token t,
choice j) with slot s = expert_map[ids[t,j]] (or the id itself without a
map), s = -1 contributing nothing,

    gate, up = W13[s][:I] @ x_t, W13[s][I:] @ x_t
    out[t]  += w[t,j] * W2[s] @ (silu(gate) * up)

accumulated in float64, then the optional routed scale and shared-expert
output are applied.  fp8 e4m3fn weights are dequantised in closed form
q * scale[row // 128, col // 128].
"""

from __future__ import annotations

import numpy as np


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return ((u >> 16) & 0xFFFF).astype(np.uint16)


def _e4m3fn_table() -> np.ndarray:
    t = np.zeros(256, dtype=np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 7
        if e == 15 and m == 7:
            t[b] = np.nan
        elif e == 0:
            t[b] = s * (m / 8.0) * 2.0 ** -6
        else:
            t[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3FN = _e4m3fn_table()


def fp8_e4m3fn_to_f32(q: np.ndarray) -> np.ndarray:
    return E4M3FN[np.asarray(q, dtype=np.uint8)]


def dequant_block(q: np.ndarray, scale: np.ndarray, block: int = 128) -> np.ndarray:
    """q [..., R, C] uint8 e4m3fn, scale [..., ceil(R/b), ceil(C/b)] -> f32."""
    w = fp8_e4m3fn_to_f32(q)
    R, C = w.shape[-2:]
    s = np.repeat(np.repeat(scale, block, axis=-2)[..., :R, :], block, axis=-1)[..., :C]
    return (w * s).astype(np.float32)


def silu(v: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):  # exp(-v) = inf for v << 0 gives the limit -0
        return v / (1.0 + np.exp(-v))


def fused_experts(x, w13, w2, topk_w, topk_ids, expert_map=None, scale: float = 1.0,
                  shared=None) -> np.ndarray:
    """x [T,H]; w13 [S,2I,H]; w2 [S,H,I]; topk_w/ids [T,k] -> out [T,H] f64."""
    x = np.asarray(x, dtype=np.float64)
    T, H = x.shape
    I = w2.shape[2]
    S = w13.shape[0]
    out = np.zeros((T, H), dtype=np.float64)
    ids = np.asarray(topk_ids)
    tw = np.asarray(topk_w, dtype=np.float64)
    # (token, choice) pairs grouped by slot so each expert's weights are
    # widened to float64 once; the per-pair arithmetic is unchanged.
    by_slot: dict[int, list[tuple[int, int]]] = {}
    for t in range(T):
        for j in range(ids.shape[1]):
            g = int(ids[t, j])
            if expert_map is not None:
                if not (0 <= g < len(expert_map)):
                    continue
                s = int(expert_map[g])
            else:
                s = g
            if not (0 <= s < S):
                continue
            by_slot.setdefault(s, []).append((t, j))
    for s, pairs in by_slot.items():
        a13 = np.asarray(w13[s], dtype=np.float64)
        a2 = np.asarray(w2[s], dtype=np.float64)
        for t, j in pairs:
            h = a13 @ x[t]
            a = silu(h[:I]) * h[I:]
            y = a2 @ a
            out[t] += tw[t, j] * y
    out *= scale
    if shared is not None:
        out += np.asarray(shared, dtype=np.float64)
    return out


def shared_mlp(x, gate_up, down) -> np.ndarray:
    """The shared experts as one SwiGLU MLP (the traced tail's
    shared_experts(x), src/sluice/offloader.py:341-342, 2602; closed form of
    TF:deepseek_v2/modeling_deepseek_v2.py DeepseekV2MLP):
    down @ (silu(gate @ x_t) * (up @ x_t)), gate_up [2*Is, H] holding the
    gate rows then the up rows, down [H, Is] -> [T, H] float64."""
    x = np.asarray(x, dtype=np.float64)
    gu = np.asarray(gate_up, dtype=np.float64)
    d = np.asarray(down, dtype=np.float64)
    Is = d.shape[1]
    h = x @ gu.T
    return (silu(h[:, :Is]) * h[:, Is:]) @ d.T


def rel_l2(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


def align_blocks(topk_ids, expert_map, S: int, block_m: int = 16):
    """Reference grouping of (token, choice) pairs by slot: list of
    (slot, [pairs]) blocks, slots ascending, pairs ascending, <= block_m per
    block; and the per-pair validity list."""
    ids = np.asarray(topk_ids).reshape(-1)
    E = len(expert_map) if expert_map is not None else None
    per_slot: dict[int, list[int]] = {}
    valid = []
    for p, g in enumerate(ids):
        g = int(g)
        s = -1
        if expert_map is None:
            s = g
        elif 0 <= g < E:
            s = int(expert_map[g])
        if not (0 <= s < S):
            valid.append(0)
            continue
        valid.append(1)
        per_slot.setdefault(s, []).append(p)
    blocks = []
    for s in sorted(per_slot):
        ps = per_slot[s]
        for i in range(0, len(ps), block_m):
            blocks.append((s, ps[i:i + block_m]))
    return blocks, valid
