"""The synthetic inputs of the benchmark configurations, generated on the device.

Every input is a function of a seed through rng::derive(seed, "<config>/<tensor>") streams
(src/rng.rs:9-17) and the element index (include/noetic_synth.h), so a configuration is
reproducible on any box. Configurations (BASELINE.json `configs`):

  c2  decode step: f32 [1,64,1,32000] ~ N(0,1) with 8 spike tokens per row raised by +6;
      no mask; temperature 0.8; outputs ids + logp.
  c3  PPO scoring: bf16 policy [8,16,512,50304] ~ N(0,1.5^2); bf16 reference = RNE(policy +
      N(0,0.1^2)); target tokens uniform in [0,V); outputs logp, ref logp, exact KL, k1/k2/k3,
      entropy.
  c4  constrained decode (north star): bf16 [1,256,1,128256] ~ N(0,2^2); u8 grammar-like mask
      [256,V] of contiguous kept runs (mean 96) between excluded gaps (mean 224), about 30% kept,
      at least one per row; temperature 0.7; outputs ids + logp.
  c5  large-vocab scoring: f32 [4,32,1024,151936] ~ N(0,1) with a Zipf(1.1) rank bias
      -1.1*ln(1 + rank), rank = (v + rot_row) mod V; u8 mask Bernoulli(0.9) per element with the
      scored token always kept; tokens uniform in [0,V); outputs logp, entropy, and group
      advantages over groups of 8 along B of the per-sequence mean log-probability.
`rows` arguments shrink a configuration for a test (the row shape is unchanged).
"""
import ctypes as C

import numpy as np

import noetic_rl as nr


def _key(seed, label):
    return nr.Rng(seed, label).key()


def normal(shape, dtype, seed, label, std=1.0, mean=0.0, zipf=0.0, base=None):
    rows, V = int(np.prod(shape[:-1])), shape[-1]
    t = nr.Tensor(shape, dtype)
    a = nr.NtSynthNormal(t.ptr, nr.NT_F32 if dtype == "f32" else nr.NT_BF16, rows, V, _key(seed, label), mean, std,
                         zipf, _key(seed, label + "/rotation"), None if base is None else base.ptr)
    nr._check(nr.lib().nt_synth_normal(C.byref(a)), "synth normal")
    return t


def tokens(shape, V, seed, label):
    t = nr.IntTensor(shape)
    nr._check(nr.lib().nt_synth_tokens(t.ptr, t.numel, _key(seed, label), V), "synth tokens")
    return t


def c2(seed=2024, rows=64):
    V = 32000
    x = normal((1, rows, 1, V), "f32", seed, "c2/logits")
    nr._check(nr.lib().nt_synth_spikes(x.ptr, nr.NT_F32, rows, V, 8, _key(seed, "c2/spikes"), 6.0), "spikes")
    return {"name": "c2", "logits": x, "mask": None, "temperature": 0.8, "rows": rows, "V": V}


def c4(seed=2024, rows=256, shared_mask=False):
    """C4's decode rows; with shared_mask, one grammar mask [1, V] that every row reads (mask_ld 0)."""
    V = 128256
    x = normal((1, rows, 1, V), "bf16", seed, "c4/logits", std=2.0)
    mrows = 1 if shared_mask else rows
    m = np.empty((1, mrows, 1, V), dtype=np.uint8)
    lab = b"c4/mask"
    nr._check(nr.lib().nt_synth_runs_mask_host(m.ctypes.data_as(C.c_void_p), mrows, V, seed, lab, len(lab), 96, 224),
              "runs mask")
    return {"name": "c4s" if shared_mask else "c4", "logits": x, "mask": nr.Tensor.from_numpy(m, "u8"),
            "mask_shared": shared_mask, "temperature": 0.7, "rows": rows, "V": V}


def c3(seed=2024, rows=8 * 16 * 512):
    V = 50304
    shape = (rows, V) if rows != 8 * 16 * 512 else (8, 16, 512, V)
    pol = normal(shape, "bf16", seed, "c3/policy", std=1.5)
    ref = normal(shape, "bf16", seed, "c3/reference_noise", std=0.1, base=pol)
    tok = tokens(shape[:-1], V, seed, "c3/tokens")
    return {"name": "c3", "logits": pol, "ref": ref, "tokens": tok, "temperature": 1.0, "rows": rows, "V": V}


def c5(seed=2024, rows=4 * 32 * 1024):
    V = 151936
    shape = (rows, V) if rows != 4 * 32 * 1024 else (4, 32, 1024, V)
    x = normal(shape, "f32", seed, "c5/logits", zipf=1.1)
    m = nr.Tensor(shape, "u8")
    nr._check(nr.lib().nt_synth_bernoulli_mask(m.ptr, m.numel, _key(seed, "c5/mask"), 0.9), "bernoulli")
    tok = tokens(shape[:-1], V, seed, "c5/tokens")
    nr._check(nr.lib().nt_synth_keep_tokens(m.ptr, rows, V, tok.ptr), "keep tokens")
    return {"name": "c5", "logits": x, "mask": m, "tokens": tok, "temperature": 1.0, "rows": rows, "V": V}


def download_rows(t, row_ids, V):
    """The exact bytes of selected rows of a [rows, V] device tensor (for the CPU oracle)."""
    itemsize = np.dtype(nr._NP[t.dtype]).itemsize
    out = np.empty((len(row_ids), V), dtype=nr._NP[t.dtype])
    for i, r in enumerate(row_ids):
        nr._check(nr.lib().nt_hip_download(out[i].ctypes.data_as(C.c_void_p),
                                           C.c_void_p(t.ptr + int(r) * V * itemsize), V * itemsize), "download row")
    return out


def bf16_to_f32(a):
    return (a.astype(np.uint32) << 16).view(np.float32)
