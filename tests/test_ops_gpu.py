"""The non-matvec ComputeBackend methods on the GPU, read like the
reference's CpuBackend tests (yule-gpu/src/cpu.rs:597-1157): known answers
from those tests (tests/golden/reference_kats.json) plus float64 numpy
references on seeded inputs."""
import math
import sys

import numpy as np
import pytest

import oracle
from refgen import kats
from yule_amd import synth
from yule_amd.backend import YuleGpuError

pytestmark = pytest.mark.gpu
K = kats()


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def f32(a):
    return np.asarray(a, dtype=np.float32)


def close(a, b, tol):
    return np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))) <= tol


def test_allocate_zeroed_and_copies(hip):
    say("[ops] allocate / copies")
    h = hip.allocate(64)
    assert np.all(hip.download(h, 16) == 0)                        # cpu.rs:157 zero-initialised
    src, dst = hip.upload(f32([1, 2, 3, 4])), hip.allocate(16)
    hip.copy_buffer(src, dst, 16)
    assert list(hip.download(dst, 4)) == [1, 2, 3, 4]
    cache = hip.allocate(4 * 4 * 4)                                 # KV-cache write pattern (cpu.rs:805-857)
    hip.copy_buffer_offset(src, cache, 0, 2 * 16, 16)
    got = hip.download(cache, 16)
    assert list(got[8:12]) == [1, 2, 3, 4] and np.all(got[:8] == 0) and np.all(got[12:] == 0)
    with pytest.raises(YuleGpuError):
        hip.copy_buffer_offset(src, cache, 0, 60, 16)              # past the end of dst
    with pytest.raises(YuleGpuError):
        hip.copy_to_device(np.zeros(32, np.float32), src)          # larger than the buffer
    for b in (h, src, dst, cache):
        hip.free(b)
    hip.free(h)                                                     # unknown handles are ignored (cpu.rs free)


def test_rms_norm_softmax_elementwise(hip):
    say("[ops] rms_norm / softmax / silu / mul / add / silu_mul")
    n = 2048
    x, w, b = synth.gauss(1, n), synth.gauss(2, n), synth.gauss(3, n)
    hx, hw, hb, ho = hip.upload(x), hip.upload(w), hip.upload(b), hip.allocate(4 * n)
    xd, wd, bd = x.astype(np.float64), w.astype(np.float64), b.astype(np.float64)
    hip.rms_norm(hx, hw, ho, n, 1e-5)
    assert close(hip.download(ho, n), xd / np.sqrt(np.mean(xd * xd) + 1e-5) * wd, 1e-5)
    hip.softmax(hx, ho, n)
    e = np.exp(xd - xd.max())
    assert close(hip.download(ho, n), e / e.sum(), 1e-7)
    hip.silu(hx, ho, n)
    assert close(hip.download(ho, n), xd / (1 + np.exp(-xd)), 1e-6)
    hip.element_mul(hx, hb, ho, n)
    assert close(hip.download(ho, n), xd * bd, 1e-6)
    hip.add(hx, hb, ho, n)
    assert close(hip.download(ho, n), xd + bd, 1e-6)
    hip.silu_mul(hx, hb, ho, n)
    assert close(hip.download(ho, n), xd / (1 + np.exp(-xd)) * bd, 1e-5)
    for h in (hx, hw, hb, ho):
        hip.free(h)


def test_rope_kats_and_table(hip):
    say("[ops] rope")
    k0 = K["rope_pos0"]
    q, k = hip.upload(f32(k0["q"])), hip.upload(f32(k0["k"]))
    hip.rope(q, k, 0, 4, 10000.0, 1, 1)
    assert close(hip.download(q, 4), k0["expect_q"], 1e-5) and close(hip.download(k, 4), k0["expect_k"], 1e-5)
    hip.copy_to_device(f32(K["rope_pos5"]["q"]), q)
    hip.rope(q, k, 5, 4, 10000.0, 1, 1)
    got = hip.download(q, 4)
    assert abs(got[0] - math.cos(5.0)) < 1e-4 and abs(got[1] - math.sin(5.0)) < 1e-4
    # many heads, many positions vs the oracle's RopeTable (model_runner.rs:77-100)
    hd, nq, nk, pos = 64, 32, 4, 300
    qv, kv = synth.gauss(4, nq * hd), synth.gauss(5, nk * hd)
    hq, hk = hip.upload(qv), hip.upload(kv)
    hip.rope(hq, hk, pos, hd, 10000.0, nq, nk)
    c, s = oracle.rope_table(pos + 1, hd, 10000.0)
    c, s = c[pos * 32:(pos + 1) * 32], s[pos * 32:(pos + 1) * 32]

    def rot(v):
        v = v.reshape(-1, hd).astype(np.float64)
        o = v.copy()
        o[:, 0::2] = v[:, 0::2] * c - v[:, 1::2] * s
        o[:, 1::2] = v[:, 0::2] * s + v[:, 1::2] * c
        return o.reshape(-1)
    # device trig vs host libm: both round the same f32 formula; 1e-4 absolute on |x| ~ 3
    assert close(hip.download(hq, nq * hd), rot(qv), 1e-4) and close(hip.download(hk, nk * hd), rot(kv), 1e-4)
    for h in (q, k, hq, hk):
        hip.free(h)


def test_matmul_f32(hip):
    say("[ops] matmul")
    m, n, k = 3, 70, 129
    a, b = synth.gauss(6, (m, k)), synth.gauss(7, (k, n))
    ha, hb, hc = hip.upload(a), hip.upload(b), hip.allocate(4 * m * n)
    hip.matmul(ha, hb, hc, m, n, k)
    assert close(hip.download(hc, (m, n)), a.astype(np.float64) @ b.astype(np.float64), 1e-4)
    for h in (ha, hb, hc):
        hip.free(h)


def test_attn_score_value_kats(hip):
    say("[ops] attn_score / attn_value")
    a = K["attn_score"]
    q, kc, vc = hip.upload(f32(a["q"])), hip.upload(f32(a["k_cache"])), hip.upload(f32(a["v_cache"]))
    sc, out = hip.allocate(4 * 3), hip.allocate(4 * 8)
    hip.attn_score(q, kc, sc, 2, 3, 0, 0, 4)
    s = hip.download(sc, 3)
    assert close(s * math.sqrt(2), a["expect_scores_times_sqrt2"], 1e-5)
    hip.softmax(sc, sc, 3)
    hip.attn_value(sc, vc, out, 2, 3, 0, 4, 0)
    p = hip.download(sc, 3).astype(np.float64)
    V = np.array(a["v_cache"]).reshape(3, 4)[:, :2]
    assert close(hip.download(out, 2), p @ V, 1e-4)
    for h in (q, kc, vc, sc, out):
        hip.free(h)


@pytest.mark.parametrize("hd,nh,nkv,seq", [(2, 2, 1, 2), (64, 32, 4, 384), (128, 32, 8, 1000), (64, 8, 8, 1),
                                          (256, 8, 2, 200), (64, 32, 4, 600), (80, 8, 2, 77), (32, 4, 4, 33),
                                          (16, 8, 2, 100), (8, 4, 1, 50), (4, 4, 2, 300), (48, 8, 2, 200),
                                          (4, 32, 2, 1500), (16, 32, 2, 3000), (96, 32, 2, 1100)])
def test_gqa_decode_attn(hip, hd, nh, nkv, seq):
    say(f"[ops] gqa_decode_attn hd={hd} heads={nh}/{nkv} seq={seq}")
    if hd == 2:
        g = K["gqa_2to1"]
        q, kc, vc = f32(g["q"]), f32(g["k_cache"]), f32(g["v_cache"])
        with pytest.raises(YuleGpuError):           # head_dim must be a multiple of 4 here
            hip.gqa_decode_attn(hip.upload(q), hip.upload(kc), hip.upload(vc), hip.allocate(16), 2, 1, 2, 2)
        return
    run_gqa_case(hip, hd, nh, nkv, seq)


def gqa_ref(q, kc, vc, nh, nkv, hd):
    want = np.zeros(nh * hd)
    for h in range(nh):
        kv = h // (nh // nkv)
        Kh = kc[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        s = Kh @ q[h * hd:(h + 1) * hd] / math.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        want[h * hd:(h + 1) * hd] = p @ vc[:, kv * hd:(kv + 1) * hd]
    return want


def run_gqa_case(hip, hd, nh, nkv, seq, tol=1e-5):
    q, kc, vc = synth.gauss(8, nh * hd), synth.gauss(9, (seq, nkv * hd)), synth.gauss(10, (seq, nkv * hd))
    hq, hk, hv, ho = hip.upload(q), hip.upload(kc), hip.upload(vc), hip.allocate(4 * nh * hd)
    hip.gqa_decode_attn(hq, hk, hv, ho, nh, nkv, hd, seq)
    got = hip.download(ho, nh * hd)
    for h in (hq, hk, hv, ho):
        hip.free(h)
    want = gqa_ref(q, kc, vc, nh, nkv, hd)
    err = np.max(np.abs(got - want))
    assert err <= tol, f"max error {err:.3g}"


@pytest.mark.parametrize("hd,nh,nkv,seq", [(64, 8, 2, 1), (64, 8, 2, 65), (64, 32, 4, 384), (128, 32, 8, 1000),
                                          (80, 8, 2, 77), (32, 4, 4, 33), (64, 24, 8, 300), (64, 40, 8, 500),
                                          (256, 16, 2, 129), (128, 56, 8, 257), (64, 4, 4, 700)])
def test_gqa_decode_attn_split_forced(hip, hd, nh, nkv, seq, monkeypatch):
    """The split-KV path (per-chunk max / sum / partial output, then the
    combine) at every group size 1..8 and every chunk length, forced on
    short sequences."""
    say(f"[ops] split gqa_decode_attn hd={hd} heads={nh}/{nkv} seq={seq}")
    monkeypatch.setenv("YULE_ATTN_SPLIT_MIN", "1")
    run_gqa_case(hip, hd, nh, nkv, seq)


@pytest.mark.parametrize("hd,nh,nkv,seq", [(64, 32, 4, 5000), (128, 32, 8, 9000), (64, 32, 4, 20000),
                                          (128, 64, 8, 17000)])
def test_gqa_decode_attn_long(hip, hd, nh, nkv, seq):
    """Long contexts: split-KV by default from 512 positions; above 16384
    (the one-workgroup-per-head kernel's LDS limit) it is the only path."""
    say(f"[ops] long gqa_decode_attn hd={hd} heads={nh}/{nkv} seq={seq}")
    run_gqa_case(hip, hd, nh, nkv, seq)


def test_gqa_decode_attn_limits(hip):
    """More than 8 query heads per KV head: the per-head kernel up to 16384
    positions, refused above; above 262144 positions refused for any shape."""
    say("[ops] gqa_decode_attn limits")
    run_gqa_case(hip, 64, 32, 2, 2000)
    h = hip.allocate(4 * 64 * 32)
    with pytest.raises(YuleGpuError, match="8 query heads"):
        hip.gqa_decode_attn(h, h, h, h, 32, 2, 64, 16385)
    with pytest.raises(YuleGpuError, match="262144"):
        hip.gqa_decode_attn(h, h, h, h, 32, 4, 64, 262145)
    with pytest.raises(YuleGpuError, match="131072"):   # per-head kernel's cache row width
        hip.gqa_decode_attn(h, h, h, h, 513, 513, 256, 10)
    hip.free(h)


def test_argmax_kats(hip):
    say("[ops] argmax")
    out = hip.allocate(4)
    for vals, want in ((K["argmax"]["values"], K["argmax"]["expect"]), ([1.0, 3.0, 3.0, 2.0], 2),
                       ([5.0] * 3000, 2999)):
        h = hip.upload(f32(vals))
        hip.argmax(h, len(vals), out)
        assert int(hip.download(out, 1, np.uint32)[0]) == want
        hip.free(h)
    v = synth.gauss(11, 32000)
    h = hip.upload(v)
    hip.argmax(h, 32000, out)
    assert int(hip.download(out, 1, np.uint32)[0]) == oracle.argmax(v)
    hip.free(h)
    # ties between infinities: argmax_ct's sign test keeps the first (inf - inf
    # is a negative NaN on x86), equal finite maxima go to the last; the oracle
    # runs the reference's scan
    inf = np.inf
    cases = [[inf, 1.0, inf], [-inf] * 5, [1.0, inf, 2.0, inf], [-inf, 3.0, 3.0], [2.0, -inf],
             [-inf, -inf, 0.5, -inf], [inf] * 4000]
    big = np.full(5000, -inf, np.float32)
    big[[17, 2500, 4999]] = inf
    cases.append(big)
    for vals in cases:
        a = f32(vals)
        want = oracle.argmax(a)
        h = hip.upload(a)
        hip.argmax(h, len(a), out)
        assert int(hip.download(out, 1, np.uint32)[0]) == want, vals
        hip.free(h)
    hip.free(out)


@pytest.mark.parametrize("pattern", [0, 1, 2])
@pytest.mark.parametrize("loads", [1, 2, 4, 8])
def test_read_probe_variants_read_every_word_once(hip, pattern, loads):
    """Each read-probe variant covers every word exactly once, at ragged
    sizes and grids that leave lanes, runs and chunks partly empty."""
    say(f"[ops] read_probe_variant pattern {pattern}, {loads} loads in flight")
    for n_bytes, n_wg in ((16, 1), (16, 64), (4096, 3), (1_000_016, 2048), (33_030_144, 1024)):
        data = np.random.default_rng(n_bytes + loads).integers(0, 2**32, n_bytes // 4, dtype=np.uint32)
        src, part = hip.upload(data), hip.allocate(4 * n_wg)
        hip.read_probe_variant(src, n_bytes, part, n_wg, pattern, loads)
        got = np.bitwise_xor.reduce(hip.download(part, n_wg, np.uint32))
        assert int(got) == int(np.bitwise_xor.reduce(data)), (n_bytes, n_wg)
        hip.free(src)
        hip.free(part)
    src, part = hip.allocate(64), hip.allocate(4)
    with pytest.raises(YuleGpuError):
        hip.read_probe_variant(src, 64, part, 1, 3, loads)    # no such pattern
    with pytest.raises(YuleGpuError):
        hip.read_probe_variant(src, 64, part, 1, pattern, 3)  # loads not a power of two up to 8
    hip.free(src)
    hip.free(part)


@pytest.mark.parametrize("n_bytes,n_wg", [(16, 1), (16, 64), (4096, 3), (1_000_016, 2048), (33_030_144, 2048)])
def test_read_probe_reads_every_word_once(hip, n_bytes, n_wg):
    """The roofline probe: the XOR of its per-workgroup partials equals the
    XOR of every 32-bit word of the range (each word read exactly once)."""
    say(f"[ops] read_probe {n_bytes} B over {n_wg} workgroups")
    rng = np.random.default_rng(n_bytes)
    data = rng.integers(0, 2**32, n_bytes // 4, dtype=np.uint32)
    src, part = hip.upload(data), hip.allocate(4 * n_wg)
    hip.read_probe(src, n_bytes, part, n_wg)
    got = np.bitwise_xor.reduce(hip.download(part, n_wg, np.uint32))
    assert int(got) == int(np.bitwise_xor.reduce(data))
    with pytest.raises(YuleGpuError):
        hip.read_probe(src, n_bytes + 16, part, n_wg)          # past the buffer
    with pytest.raises(YuleGpuError):
        hip.read_probe(src, n_bytes - 4 if n_bytes > 16 else 8, part, n_wg)   # not a multiple of 16
    with pytest.raises(YuleGpuError):
        hip.read_probe(src, n_bytes, part, n_wg + 1)           # partials too small
    hip.free(src)
    hip.free(part)
