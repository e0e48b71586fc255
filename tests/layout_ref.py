"""Test-side restatement of the packed slot layout (independent of the kernels), used to read
packed buffers back into natural token order."""
import torch


def slot_tokens(frames, tokens_per_frame, num_special):
    """Token id of every packed slot (-1 for padding)."""
    T, ns = tokens_per_frame, num_special
    P = T - ns
    nbf = -(-P // 64)
    S = frames * ns
    Sp = -(-S // 64) * 64
    toks = [-1] * (Sp + frames * nbf * 64)
    for s in range(S):
        toks[s] = (s // ns) * T + s % ns
    for f in range(frames):
        for p in range(P):
            toks[Sp + f * nbf * 64 + p] = f * T + ns + p
    return torch.tensor(toks, dtype=torch.long)


def framed_slot_tokens(frames, tokens_per_frame, num_special):
    """Token id of every slot of a head in the framed layout (-1 for padding), over the same number of
    slots as the packed layout: frame f's tokens in order from slot 64 * ceil(T/64) * f."""
    T = tokens_per_frame
    nslots = len(slot_tokens(frames, tokens_per_frame, num_special))
    tp = -(-T // 64) * 64
    toks = [-1] * nslots
    for f in range(frames):
        for t in range(T):
            toks[f * tp + t] = f * T + t
    return torch.tensor(toks, dtype=torch.long)


def kappa(c):
    return (c & ~12) | ((c & 4) << 1) | ((c & 8) >> 1)


def phi(i):
    return 16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3)


def unpack_rows(packed, toks, n_tokens):
    """[H, L, 64] packed rows -> [H, N, 64] natural rows; also returns the padding rows."""
    H = packed.shape[0]
    out = torch.zeros(H, n_tokens, packed.shape[-1], dtype=packed.dtype)
    valid = toks >= 0
    out[:, toks[valid]] = packed[:, valid]
    return out, packed[:, ~valid]


def unpack_v(vt, toks, n_tokens):
    """[H, L/64, 64, 64] transposed tiles -> [H, N, 64] natural rows (and the padding rows)."""
    H, nt = vt.shape[:2]
    perm_c = torch.tensor([kappa(c) for c in range(64)])
    d_of_row = torch.tensor([32 * (i // 32) + phi(i % 32) for i in range(64)])
    rows = torch.empty(H, nt, 64, 64, dtype=vt.dtype)  # [H, tile, slot-in-tile, d]
    # tile[i][c] = V[64*tile + kappa(c)][d_of_row[i]]
    rows[:, :, perm_c[None, :].expand(64, 64), d_of_row[:, None].expand(64, 64)] = vt
    rows = rows.reshape(H, nt * 64, 64)
    return unpack_rows(rows, toks, n_tokens)
