"""The DK = 128 chunk-local stage on its own: the factored transition records
it writes (csrc/gdn2_prefill_layout.h) against the same matrices formed in
float64 from their definitions (reference gdn2/reference.py:116-197 for Aqk,
Akk, Ai and the WY factors; the record products as the scan uses them):

    E = b k gamma,  MOZ = Aqk Ai,  KA = KG^T Ai,  QP = Qg - MOZ E,  gamma_last,

and the transition's rank-64 product M = KA E formed from the decoded E and
KA, against M from the float64 factors.

Every matrix is stored as fp16 (11-bit significand) after products of fp16
operands, so each is held to 3e-3 of its own largest entry, plus an absolute
2^-22 (four steps of fp16's subnormal spacing) for entries below fp16's
normal range: with strong decay the whole of E is ~1e-19 (a full chunk of
decay) and is stored as zeros, which moves the state by less than 2^-17 of
its own scale per chunk. Inputs are fp32
and cover every path of the kernel's decay handling: small decay (fp16
off-diagonal blocks, split-bf16 diagonal), the test suite's default decay
scale 4, and decay scale 30, where a 16-token block's decay spread exceeds
the split operands' range and the diagonal block is summed exactly."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from gdt2_tilelang_amd import _hip


DK = 128
FRAG = 512
# factored chunk record (16-bit offsets): E, KA, QP, MOZ fragments, gamma_last, scales
E_OFF, KA_OFF, QP_OFF, MOZ_OFF, GL_OFF, SC_OFF, STRIDE = 0, 8192, 16384, 24576, 28672, 28928, 29056


def frags_to_matrix(rec, off, mt, kt):
    """fp16 A-operand fragments [mt][kt] -> a [16 mt, 32 kt] matrix (lane
    16 lq + lr holds row lr, columns 8 lq .. 8 lq + 7 of its 16 x 32 tile)."""
    f = rec[off:off + mt * kt * FRAG].view(np.float16).astype(np.float64).reshape(mt, kt, 4, 16, 8)
    # [m][kk][lq][lr][j] -> rows 16 m + lr, columns 32 kk + 8 lq + j
    return f.transpose(0, 3, 1, 2, 4).reshape(16 * mt, 32 * kt)


# accumulator k order: lane group lq, element j holds k = 4 lq + j (j < 4) and
# 16 + 4 lq + j - 4 (j >= 4) within each 32-wide k step
ACC_COL = np.array([[4 * lq + j if j < 4 else 16 + 4 * lq + j - 4 for j in range(8)] for lq in range(4)])


def frags_to_matrix_acc(rec, off, mt, kt):
    """As frags_to_matrix, for fragments whose k index is in accumulator order."""
    f = rec[off:off + mt * kt * FRAG].view(np.float16).astype(np.float64).reshape(mt, kt, 4, 16, 8)
    out = np.zeros((16 * mt, 32 * kt))
    for m in range(mt):
        for kk in range(kt):
            for lq in range(4):
                out[16 * m:16 * m + 16, 32 * kk + ACC_COL[lq]] = f[m, kk, lq]
    return out


def test_accumulator_order_is_a_permutation():
    """Every column of a 32-wide k step appears once in the accumulator order,
    and lane group lq holds rows 4lq .. 4lq+3 of two consecutive 16-row
    accumulator blocks (v_mfma_f32_16x16x32: D[4 lq + e][lr])."""
    assert sorted(ACC_COL.ravel().tolist()) == list(range(32))
    for lq in range(4):
        assert ACC_COL[lq, :4].tolist() == [4 * lq + e for e in range(4)]
        assert ACC_COL[lq, 4:].tolist() == [16 + 4 * lq + e for e in range(4)]


def decode_record(rec):
    sc = rec[SC_OFF:SC_OFF + 16].view(np.float32).astype(np.float64)
    E = frags_to_matrix_acc(rec, E_OFF, 4, 4) * sc[0]
    KA = frags_to_matrix_acc(rec, KA_OFF, 8, 2) * sc[1]
    return dict(E=E, KA=KA, M=KA @ E,
                QP=frags_to_matrix(rec, QP_OFF, 4, 4) * sc[2], MOZ=frags_to_matrix(rec, MOZ_OFF, 4, 2) * sc[3],
                GL=rec[GL_OFF:GL_OFF + 256].view(np.float32).astype(np.float64))


def reference_record(q, k, g, b, scale):
    """float64 record of one 64-token chunk (arrays [64, DK])."""
    G = np.cumsum(g, axis=0)
    D = G[:, None, :] - G[None, :, :]                     # [t, s, c]
    t_ge_s = np.tril(np.ones((64, 64), dtype=bool))
    ex = np.exp(np.where(t_ge_s[:, :, None], D, -np.inf))
    aqk = scale * np.einsum("tc,sc,tsc->ts", q, k, ex)
    akk = np.einsum("tc,sc,tsc->ts", b * k, k, ex) * np.tril(np.ones((64, 64)), -1)
    ai = np.linalg.inv(np.eye(64) + akk)
    gam = np.exp(G)
    E = b * k * gam
    KG = k * np.exp(G[-1:] - G)
    Qg = scale * q * gam
    moz = aqk @ ai
    ka = KG.T @ ai
    return dict(E=E, M=ka @ E, KA=ka, QP=Qg - moz @ E, MOZ=moz, GL=np.exp(G[-1]))


def _max_rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 2.0 ** -22 / 3e-3))


@pytest.mark.gpu
@pytest.mark.parametrize("H,S", [(2, 150), (2, 2070)])
@pytest.mark.parametrize("dist,decay", [("cfg", None), ("ref", 0.3), ("ref", 4.0), ("ref", 30.0)])
def test_chunk_local_records(dist, decay, H, S):
    """S = 150: 3 chunk records, the last chunk ragged (22 rows). S = 2070: 33
    chunk records, the last ragged (22 rows)."""
    print(f"records DK=128 H={H} S={S} {dist} decay={decay}", flush=True)
    B = 1
    if dist == "cfg":
        q, k, v, g, b, w = oracle.make_config_inputs(B, S, H, DK, DK, seed=4)
    else:
        q, k, v, g, b, w = oracle.make_inputs(B, S, H, DK, DK, decay_scale=decay, seed=4)
    lib = _hip.lib()
    nbytes = lib.gdn2_hip_prefill_workspace_bytes(B, H, DK, S)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    dq, dk, dg, db = (t.cuda().contiguous() for t in (q, k, g, b))
    scale = DK ** -0.5
    rc = lib.gdn2_hip_chunk_local(_hip.ptr(dq), _hip.ptr(dk), _hip.ptr(db), _hip.ptr(dg), 0, _hip.ptr(ws), B, H,
                                  DK, S, 0, S, scale, _hip.stream_of(dq.device))
    assert rc == 0
    torch.cuda.synchronize()
    raw = ws.cpu().numpy().view(np.uint16)
    NC = (S + 63) // 64
    assert nbytes == B * H * NC * STRIDE * 2
    NR, stride = NC, STRIDE

    def chunk_ref(h, n):
        sl = slice(64 * n, min(64 * n + 64, S))
        rows = max(sl.stop - sl.start, 0)
        pad = lambda t: np.pad(t[0, sl, h].double().numpy(), ((0, 64 - rows), (0, 0)))  # noqa: E731
        return reference_record(pad(q), pad(k), pad(g), pad(b), scale)

    worst = {}
    for h in range(H):
        for n in range(NR):
            got_raw = raw[(h * NR + n) * stride:(h * NR + n + 1) * stride].copy()
            want, got = chunk_ref(h, n), decode_record(got_raw)
            for name in got:
                e = _max_rel(got[name], want[name])
                worst[name] = max(worst.get(name, 0.0), e)
    print("  " + " ".join(f"{k_}={v_:.1e}" for k_, v_ in worst.items()), flush=True)
    assert worst["GL"] < 1e-5
    for name in ("E", "M", "KA", "QP", "MOZ"):
        assert worst[name] < 3e-3, (name, worst[name])
