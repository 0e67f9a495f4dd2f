"""Helpers shared by the GPU parity tests (imported by test modules only)."""

import numpy as np

from oracle import tq_oracle as O

ATOL = 2e-3    # max-abs tolerance on attention outputs
RTOL = 1e-2    # max-rel tolerance, checked two ways below
# Element-wise max-rel: |got - want| <= RTOL * max(|want|, REL_FLOOR).  Below
# the floor the relative bar would demand more than the absolute one
# (RTOL * REL_FLOOR = ATOL), so it continues as the max-abs bar there.
REL_FLOOR = ATOL / RTOL


def assert_attn_close(got, want, atol=ATOL, rtol=RTOL, what=""):
    """The parity bar on attention outputs: max-abs <= atol, element-wise
    max-rel <= rtol (denominator floored at atol / rtol) and norm-wise
    ||got - want|| / ||want|| <= rtol."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    erel = float((err / np.maximum(np.abs(want), atol / rtol)).max()) if err.size else 0.0
    assert err.max() <= atol, f"{what} max-abs {err.max():.3e} > {atol}"
    assert erel <= rtol, f"{what} element-wise rel {erel:.3e} > {rtol}"
    assert rel <= rtol, f"{what} rel {rel:.3e} > {rtol}"
    return float(err.max()), float(rel)


def oracle_state(k, v, hot_window, vbits, seed, outlier_frac=0.02):
    """Per-sequence oracle caches for fp16 k, v (B, Hkv, L, D)."""
    D = k.shape[-1]
    pi, pi_t = O.rotation(seed, D)
    return [O.SequenceCache(hot_window=hot_window, value_bits=vbits, outlier_frac=outlier_frac)
            .build(k[b], v[b], pi, pi_t) for b in range(k.shape[0])], (pi, pi_t)


def compare_group(exp, kg, vg, what=""):
    """Exported GPU group vs oracle KeyGroup/ValueGroup, bit for bit."""
    assert np.array_equal(exp["kpacked"], kg.packed), f"{what}: key codes differ"
    assert np.array_equal(exp["nf4_scale"], kg.nf4_scale), f"{what}: nf4_scale differs"
    assert np.array_equal(exp["nf4_mean"], kg.nf4_mean), f"{what}: nf4_mean differs"
    assert np.array_equal(exp["outlier_idx"], kg.outlier_idx), f"{what}: outlier idx differ"
    assert np.array_equal(exp["outlier_val"].view(np.uint16), kg.outlier_val.view(np.uint16)), \
        f"{what}: outlier values differ"
    assert np.array_equal(exp["vpacked"], vg.packed), f"{what}: value codes differ"
    assert np.array_equal(exp["vnorms"], vg.norms), f"{what}: value norms differ"


# --------------------------------------------------------------------------- #
# Full-size checks: synthetic data on the GPU, a torch fp32  #
# dequantize-then-attend reference built on the bit-exact dequant kernel, and   #
# oracle spot checks of individual groups.                                      #
# --------------------------------------------------------------------------- #


def synth_gpu(torch, seed, B, Hkv, L, D=128):
    """fp16 keys/values (B, Hkv, L, D) on the GPU with the measurement spec's
    distribution (lognormal per-channel key scale, 2 % x10 channels, RoPE;
    N(0,1) values), generated in 4096-token chunks (bench.synth_chunk)."""
    import bench
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    scale = torch.exp(torch.randn((B, Hkv, 1, D), generator=gen, device="cuda"))
    n_hot = round(0.02 * D)
    for b in range(B):
        for h in range(Hkv):
            scale[b, h, 0, torch.randperm(D, generator=gen, device="cuda")[:n_hot]] *= 10.0
    k = torch.empty((B, Hkv, L, D), dtype=torch.float16, device="cuda")
    v = torch.empty_like(k)
    for t in range(0, L, 4096):
        n = min(4096, L - t)
        k[:, :, t:t + n], v[:, :, t:t + n] = bench.synth_chunk(torch, gen, scale, t, n, B, Hkv, D)
    return k, v


def ref_attend_gpu(torch, pool, q, b):
    """fp32 softmax(q K^T / sqrt(D)) V of sequence b over the reconstructed cache:
    dequantised coded groups (tqk_dequant_groups, bit-exact to the reference's
    decompress) followed by the fp16 hot window; GQA q-head i reads kv-head
    i // (Hq / Hkv).  Returns (Hq, D) fp32 on the GPU."""
    H, D = pool.n_kv_heads, pool.head_dim
    ng = pool.n_groups(b)
    ks, vs = [], []
    if ng:
        kk, vv = pool.dequant_groups([(b, g) for g in range(ng)])
        ks.append(kk.permute(1, 0, 2, 3).reshape(H, ng * pool.group_tokens, D))
        vs.append(vv.permute(1, 0, 2, 3).reshape(H, ng * pool.group_tokens, D))
    hk, hv = pool.hot_window_tokens(b)
    ks.append(hk.float())
    vs.append(hv.float())
    K = torch.cat(ks, 1)
    V = torch.cat(vs, 1)
    g = q.shape[-2] // H
    qf = q[b].float().reshape(H, g, D)
    s = torch.matmul(qf, K.transpose(1, 2).contiguous()) / np.sqrt(D)
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, V).reshape(H * g, D)


def check_groups_vs_oracle(pool, k, v, b, groups, pi_t, vbits, what=""):
    """Exported groups of sequence b vs the oracle's encode of the same fp16
    tokens (k, v device tensors (B, Hkv, L, D)), bit for bit."""
    G = pool.group_tokens
    _, bnd = O.polar_codebook(vbits, pool.head_dim)
    for g in groups:
        x = k[b, :, g * G:(g + 1) * G].float().cpu().numpy()
        y = v[b, :, g * G:(g + 1) * G].float().cpu().numpy()
        kg = O.encode_keys(x, pool.outlier_frac)
        vg = O.encode_values(y, pi_t, bnd, vbits)
        compare_group(pool.export_group(b, g), kg, vg, what=f"{what} seq {b} group {g}")
