"""ctypes loader of the CPU oracle (oracle/_build/libq38_oracle.so) — test infrastructure.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "libq38_oracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libq38_ref.so")

P, I32, I64, U32, U64, F32, F64 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_float, C.c_double


class Desc(C.Structure):  # field order of oracle/q38_oracle.cpp Desc
    _fields_ = [(n, C.c_int32) for n in (
        "hidden", "inter", "experts", "top_k", "gu_dim", "gu_bits", "down_dim", "down_bits",
        "gu_group", "down_group", "normalize", "has_shared", "mixed", "book_format")]


class GdnDesc(C.Structure):  # field order of oracle/q38_oracle.cpp GdnDesc
    _fields_ = [(n, C.c_int32) for n in ("hidden", "hk", "hv", "dk", "dv", "conv", "bits", "group", "fmt",
                                         "gate_silu")] + [("eps", C.c_float)]


class AttnDesc(C.Structure):  # field order of oracle/q38_oracle.cpp AttnDesc
    _fields_ = [(n, C.c_int32) for n in ("hidden", "q_heads", "kv_heads", "head_dim", "rotary_dim", "bits", "group",
                                         "fmt", "norm_offset")] + [("eps", C.c_float), ("rope_theta", C.c_double)]


class HcDesc(C.Structure):  # field order of oracle/q38_oracle.cpp HcDesc
    _fields_ = [(n, C.c_int32) for n in ("hidden", "streams", "rank", "bits", "group", "with_injection")] + [
        ("eps", C.c_float)]


def make_desc(hidden=2048, inter=512, experts=512, top_k=10, gu=(8, 14), down=(8, 14), gu_group=None,
              down_group=None, normalize=1, shared=1, mixed=0, book_format=0) -> Desc:
    return Desc(hidden, inter, experts, top_k, gu[0], gu[1], down[0], down[1], gu_group or hidden,
                down_group or inter, normalize, shared, mixed, book_format)


def _a(x):
    return x.ctypes.data_as(P)


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            subprocess.check_call(["make", "-C", os.path.join(ROOT, "oracle"), "-s"])
        self.lib = L = C.CDLL(path)
        sig = lambda n, r, *a: (setattr(getattr(L, n), "restype", r), setattr(getattr(L, n), "argtypes", list(a)))
        sig("orc_f32_to_bf16", C.c_uint16, F32)
        sig("orc_f32_to_f16", C.c_uint16, F32)
        sig("orc_f16_to_f32", F32, C.c_uint16)
        sig("orc_exp_contract", F32, F32)
        sig("orc_stream_key", U64, U64, U64, U64)
        sig("orc_bits_at", U64, U64, U64)
        sig("orc_gen_normal", None, U64, U64, U64, F64, C.c_int, P)
        sig("orc_gen_uniform_f16", None, U64, U64, U64, F64, F64, P)
        sig("orc_gen_int8", None, U64, U64, U64, P)
        sig("orc_gen_int4", None, U64, U64, U64, P)
        sig("orc_gen_code_rows", None, U64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P)
        sig("orc_gen_book", None, U64, C.c_int, C.c_int, C.c_int, P, P, P)
        sig("orc_gen_embed", None, U64, P, C.c_int, C.c_int, P)
        sig("orc_prepare_u8_book", None, P, C.c_int, C.c_int, C.c_int, P, P, P, P)
        sig("orc_packed_word_count", I64, I64, C.c_int)
        sig("orc_pack_row", C.c_int, P, I64, C.c_int, P)
        sig("orc_unpack_code", C.c_int, P, I64, I64, C.c_int, P)
        sig("orc_router_logits", None, P, C.c_int, C.c_int, P, C.c_int, P)
        sig("orc_dot_contract", F32, P, P, C.c_int)
        sig("orc_route", None, P, C.c_int, C.c_int, C.c_int, C.c_int, P, P)
        sig("orc_route_plan", C.c_int, P, C.c_int, C.c_int, C.c_int, P, P, P, P, P)
        sig("orc_moe_layer_synth", C.c_int, C.POINTER(Desc), U64, C.c_int, P, C.c_int, P, P, P, P, C.c_int)
        sig("orc_moe_layer_synth_bias", C.c_int, C.POINTER(Desc), U64, C.c_int, P, C.c_int, P, P, P, P, P,
            C.c_int)
        sig("orc_moe_layer_synth_reps", C.c_int, C.POINTER(Desc), U64, C.c_int, P, C.c_int, P, P, C.c_int,
            C.c_int, C.c_int, P)
        sig("orc_moe_layer_dense", C.c_int, C.POINTER(Desc), P, P, C.POINTER(P), C.POINTER(P), C.POINTER(P),
            P, C.c_int, P, P, P, P, C.c_int)
        sig("orc_expert_dense", C.c_int, C.POINTER(Desc), C.POINTER(P), C.POINTER(P), C.POINTER(P), C.c_int, P,
            C.c_int, P)
        sig("orc_rmsnorm", None, P, C.c_int, C.c_int, F64, P)
        sig("orc_residual_add", None, P, P, I64, P)
        sig("orc_hc_read", C.c_int, C.POINTER(HcDesc), *([P] * 10), P, C.c_int, P, P, P, P)
        sig("orc_hc_write", None, C.c_int, C.c_int, C.c_int, P, P, P, P)
        sig("orc_head_q8_synth_logits", None, U64, C.c_int, I64, I64, P, C.c_int, P, C.c_int)
        sig("orc_head_q8_logits", None, P, P, I64, C.c_int, P, C.c_int, P, C.c_int)
        sig("orc_argmax", None, P, C.c_int, I64, P, P)
        sig("orc_head_q4_synth_logits", None, U64, C.c_int, I64, I64, P, C.c_int, P, C.c_int)
        sig("orc_head_q4_logits", None, P, P, I64, C.c_int, P, C.c_int, P, C.c_int)
        sig("orc_decide_greedy", C.c_int, P, I64, P, I64, P, I64, P, P, P)
        sig("orc_plan_commit", C.c_int, U64, U64, U64, P)
        sig("orc_philox4x32_10", None, P, P, P)
        sig("orc_round_uniforms", None, U64, U64, U64, U32, P, P)
        sig("orc_accept_sampled", C.c_int, P, P, P, C.c_int, I64, F32, U64, U64, U64, P, P)
        sig("orc_plant_fault", None, C.c_int)
        sig("orc_moe_layer_dense_affine_shared", C.c_int, C.POINTER(Desc), P, P, C.POINTER(P), C.POINTER(P),
            C.POINTER(P), C.POINTER(P), C.POINTER(P), C.POINTER(P), C.c_int, C.c_int, C.c_int, C.c_int, P, C.c_int,
            P, P, P, P, C.c_int)
        sig("orc_gdn_plant_fault", None, C.c_int)
        sig("orc_gdn_recurrence", C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P, P, P, P, P, P, P, P)
        sig("orc_gdn_verify", C.c_int, C.POINTER(GdnDesc), C.POINTER(P), C.POINTER(P), C.POINTER(P), P, P, P, P, P,
            C.c_int, P, P, P)
        sig("orc_mlp_map", None, C.c_int, C.c_int, P, P, P, P, C.c_int, P)
        sig("orc_attn_plant_fault", None, C.c_int)
        sig("orc_rope_table", None, C.c_double, C.c_int, I64, P, P)
        sig("orc_attn_verify", C.c_int, C.POINTER(AttnDesc), C.POINTER(P), C.POINTER(P), C.POINTER(P), P, P, P,
            C.c_int, P, P, I64, I64, I64, P)
        sig("orc_affine_expert", C.c_int, C.POINTER(P), C.POINTER(P), C.POINTER(P), C.c_int, C.c_int, C.c_int,
            C.c_int, C.c_int, P, C.c_int, P)
        sig("orc_route_synth", C.c_int, C.POINTER(Desc), U64, C.c_int, P, C.c_int, P, P, P, P, C.c_int)

    # ---- formats
    def bf16(self, x):
        f = np.ascontiguousarray(x, dtype=np.float32)
        u = f.view(np.uint32)
        out = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
        return out

    @staticmethod
    def bf16_to_f32(u16):
        return (np.asarray(u16, dtype=np.uint32) << 16).view(np.float32)

    # ---- generator
    def key(self, seed, layer, tensor):
        return self.lib.orc_stream_key(seed, layer, tensor)

    def normal(self, key, start, count, sd, f16=False):
        out = np.empty(count, np.uint16)
        self.lib.orc_gen_normal(key, start, count, sd, int(f16), _a(out))
        return out

    def uniform_f16(self, key, start, count, lo, hi):
        out = np.empty(count, np.uint16)
        self.lib.orc_gen_uniform_f16(key, start, count, lo, hi, _a(out))
        return out

    def code_rows(self, key, e, out_dim, o0, nrows, nsub, bits):
        words = ((nsub + 31) // 32) * bits
        out = np.empty(nrows * words, np.uint32)
        self.lib.orc_gen_code_rows(key, e, out_dim, o0, nrows, nsub, bits, _a(out))
        return out.reshape(nrows, words)

    def embed(self, seed, tokens, H):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty((len(t), H), np.uint16)
        self.lib.orc_gen_embed(seed, _a(t), len(t), H, _a(out))
        return out

    # ---- geometry
    def word_count(self, n, bits):
        return self.lib.orc_packed_word_count(n, bits)

    def pack_row(self, codes, bits):
        c = np.ascontiguousarray(codes, dtype=np.uint32)
        out = np.zeros(max(self.word_count(len(c), bits), 1), np.uint32)
        assert self.lib.orc_pack_row(_a(c), len(c), bits, _a(out)) == 0
        return out[: self.word_count(len(c), bits)]

    def unpack(self, words, index, bits):
        w = np.ascontiguousarray(words, dtype=np.uint32)
        out = np.zeros(1, np.uint32)
        rc = self.lib.orc_unpack_code(_a(w), len(w), index, bits, _a(out))
        return rc, int(out[0])

    # ---- router
    def router_logits(self, x, W):
        x = np.ascontiguousarray(x, np.uint16)
        W = np.ascontiguousarray(W, np.uint16)
        M, H = x.shape
        E = W.shape[0]
        out = np.empty((M, E), np.float32)
        self.lib.orc_router_logits(_a(x), M, H, _a(W), E, _a(out))
        return out

    def route(self, logits, k, normalize=1):
        lg = np.ascontiguousarray(logits, np.float32)
        M, E = lg.shape
        ex = np.empty((M, k), np.int32)
        wt = np.empty((M, k), np.float32)
        self.lib.orc_route(_a(lg), M, E, k, normalize, _a(ex), _a(wt))
        return ex, wt

    def plan(self, experts, E):
        ex = np.ascontiguousarray(experts, np.int32)
        M, k = ex.shape
        MK = M * k
        nu = np.zeros(1, np.int32)
        uexp = np.zeros(MK, np.int32)
        uoff = np.zeros(MK + 1, np.int32)
        rl = np.zeros(MK, np.int32)
        rp = np.zeros(MK, np.int32)
        assert self.lib.orc_route_plan(_a(ex), M, k, E, _a(nu), _a(uexp), _a(uoff), _a(rl), _a(rp)) == 0
        n = int(nu[0])
        return n, uexp[:n], uoff[: n + 1], rl, rp

    # ---- MoE
    def moe_layer_synth(self, d: Desc, seed, layer, x, threads=8, bias=None):
        """Synthetic layer (seed, layer) on x; bias: optional [E] float32 router-logit bias."""
        x = np.ascontiguousarray(x, np.uint16)
        M = x.shape[0]
        y = np.empty_like(x)
        ex = np.empty((M, d.top_k), np.int32)
        wt = np.empty((M, d.top_k), np.float32)
        lg = np.empty((M, d.experts), np.float32)
        if bias is None:
            rc = self.lib.orc_moe_layer_synth(C.byref(d), seed, layer, _a(x), M, _a(y), _a(ex), _a(wt), _a(lg),
                                              threads)
        else:
            b = np.ascontiguousarray(bias, np.float32)
            assert b.shape == (d.experts,)
            rc = self.lib.orc_moe_layer_synth_bias(C.byref(d), seed, layer, _a(x), M, _a(b), _a(y), _a(ex), _a(wt),
                                                   _a(lg), threads)
        assert rc == 0
        return y, ex, wt, lg

    def route_synth(self, d: Desc, seed, layer, x, threads=8, bias=None):
        """Routing alone of the synthetic layer (seed, layer) on x -> (experts, weights, logits)."""
        x = np.ascontiguousarray(x, np.uint16)
        M = x.shape[0]
        ex = np.empty((M, d.top_k), np.int32)
        wt = np.empty((M, d.top_k), np.float32)
        lg = np.empty((M, d.experts), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        rc = self.lib.orc_route_synth(C.byref(d), seed, layer, _a(x), M, None if b is None else _a(b), _a(ex),
                                      _a(wt), _a(lg), threads)
        assert rc == 0
        return ex, wt, lg

    def moe_layer_synth_reps(self, d: Desc, seed, layer, x, threads=(8,), warm=2, reps=20):
        """Seconds per pass, [len(threads), reps], of one synthetic layer (experts generated once)."""
        x = np.ascontiguousarray(x, np.uint16)
        y = np.empty_like(x)
        th = np.asarray(threads, np.int32)
        sec = np.zeros((len(th), reps), np.float64)
        assert self.lib.orc_moe_layer_synth_reps(C.byref(d), seed, layer, _a(x), x.shape[0], _a(y), _a(th),
                                                 len(th), warm, reps, _a(sec)) == 0
        return y, sec

    def moe_layer_dense(self, d: Desc, router, wsg, codes, scales, books, x, threads=8):
        x = np.ascontiguousarray(x, np.uint16)
        M = x.shape[0]
        y = np.empty_like(x)
        ex = np.empty((M, d.top_k), np.int32)
        wt = np.empty((M, d.top_k), np.float32)
        lg = np.empty((M, d.experts), np.float32)
        keep = [np.ascontiguousarray(a) for a in (router, wsg, *codes, *scales, *books)]
        arr = lambda xs: (P * 3)(*[_a(a).value for a in xs])
        rc = self.lib.orc_moe_layer_dense(C.byref(d), _a(keep[0]), _a(keep[1]), arr(keep[2:5]), arr(keep[5:8]),
                                          arr(keep[8:11]), _a(x), M, _a(y), _a(ex), _a(wt), _a(lg), threads)
        assert rc == 0
        return y, ex, wt, lg

    @staticmethod
    def _ptrs(arrs, n=3):
        return (P * n)(*[_a(a) for a in arrs])

    def gdn_plant_fault(self, code):
        self.lib.orc_gdn_plant_fault(code)

    def gdn_recurrence(self, HK, q, k, v, decay, beta, state=None):
        """The GDN recurrence alone: q, k [S, HK, DK], v [S, HV, DV], decay / beta [S, HV] as
        float32 (bf16 values), state [HV, DV, DK] bf16 bits or None -> (y [S, HV, DV] float32,
        states [S, HV, DV, DK] bf16 bits)."""
        q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
        decay, beta = np.ascontiguousarray(decay, np.float32), np.ascontiguousarray(beta, np.float32)
        S, HV, DV = v.shape
        DK = q.shape[2]
        y = np.empty((S, HV, DV), np.float32)
        st = np.empty((S, HV, DV, DK), np.uint16)
        sp = None if state is None else np.ascontiguousarray(state, np.uint16)
        rc = self.lib.orc_gdn_recurrence(HK, HV, DK, DV, S, _a(q), _a(k), _a(v), _a(decay), _a(beta),
                                         None if sp is None else _a(sp), _a(y), _a(st))
        assert rc == 0
        return y, st

    def gdn_verify(self, layer, x, origin=None):
        """GatedDeltaNet::forward_verify on rows x [S, hidden] (bf16 bits) from origin (a state
        of layer.state_elems bf16, or None for zeros) -> (out [S, hidden] bf16, checkpoints
        [S, state_elems] bf16)."""
        d = layer.odesc
        x = np.ascontiguousarray(x, np.uint16)
        S = x.shape[0]
        keep = [[np.ascontiguousarray(a) for a in layer.proj[k]] for k in ("w", "s", "b")]
        out = np.empty((S, d.hidden), np.uint16)
        ck = np.empty((S, layer.state_elems), np.uint16)
        org = None if origin is None else np.ascontiguousarray(origin, np.uint16)
        rc = self.lib.orc_gdn_verify(C.byref(d), self._ptrs(keep[0], 5), self._ptrs(keep[1], 5),
                                     self._ptrs(keep[2], 5), _a(layer.conv_w), _a(layer.a_log), _a(layer.dt_bias),
                                     _a(layer.norm_w), _a(x), S, None if org is None else _a(org), _a(out), _a(ck))
        assert rc == 0
        return out, ck

    def mlp_map(self, y, full=None, left=None, right=None):
        """The decoder's MLP output map on rows y [rows, H] (bf16 bits): the full map [H, H] or the
        low-rank pair left [H, R], right [R, H] (bf16 bits) -> out [rows, H] bf16 bits."""
        y = np.ascontiguousarray(y, np.uint16)
        rows, H = y.shape
        rank = 0 if full is not None else left.shape[1]
        keep = [None if a is None else np.ascontiguousarray(a, np.uint16) for a in (full, left, right)]
        out = np.empty_like(y)
        self.lib.orc_mlp_map(H, rank, *[None if a is None else _a(a) for a in keep], _a(y), rows, _a(out))
        return out

    def attn_plant_fault(self, code):
        self.lib.orc_attn_plant_fault(code)

    def rope_table(self, theta, R, pos):
        c = np.empty(R // 2, np.float32)
        sn = np.empty(R // 2, np.float32)
        self.lib.orc_rope_table(theta, R, pos, _a(c), _a(sn))
        return c, sn

    def attn_verify(self, layer, x, keys, values, T0, position):
        """SelfAttention::forward_verify (dense) on rows x [S, hidden] (bf16 bits) over a cache
        keys / values [HKV, cap, D] (bf16 bits, T0 tokens valid) -> (out [S, hidden] bf16,
        keys, values after the call: copies with the S new rows at T0..T0+S-1)."""
        d = layer.odesc
        x = np.ascontiguousarray(x, np.uint16)
        S = x.shape[0]
        k2, v2 = np.array(keys, np.uint16, copy=True, order="C"), np.array(values, np.uint16, copy=True, order="C")
        cap = k2.shape[1]
        keep = [[np.ascontiguousarray(a) for a in layer.proj[k]] for k in ("w", "s", "b")]
        out = np.empty((S, d.hidden), np.uint16)
        rc = self.lib.orc_attn_verify(C.byref(d), self._ptrs(keep[0], 4), self._ptrs(keep[1], 4),
                                      self._ptrs(keep[2], 4), _a(layer.q_norm), _a(layer.k_norm), _a(x), S,
                                      _a(k2), _a(v2), cap, T0, position, _a(out))
        assert rc == 0
        return out, k2, v2

    def affine_expert(self, sa, x):
        """The affine shared expert (sa: dict with w, s, b lists of 3 arrays, bits, group, inter,
        fmt) on rows of x -> T(down) [M, H] float32."""
        x = np.ascontiguousarray(x, np.uint16)
        M, H = x.shape
        keep = [[np.ascontiguousarray(a) for a in sa[k]] for k in ("w", "s", "b")]
        out = np.empty((M, H), np.float32)
        rc = self.lib.orc_affine_expert(self._ptrs(keep[0]), self._ptrs(keep[1]), self._ptrs(keep[2]), H, sa["inter"],
                                        sa["bits"], sa["group"], sa["fmt"], _a(x), M, _a(out))
        assert rc == 0
        return out

    def moe_layer_dense_affine_shared(self, d: Desc, router, wsg, codes, scales, books, sa, x, threads=8):
        x = np.ascontiguousarray(x, np.uint16)
        M = x.shape[0]
        y = np.empty_like(x)
        ex = np.empty((M, d.top_k), np.int32)
        wt = np.empty((M, d.top_k), np.float32)
        lg = np.empty((M, d.experts), np.float32)
        keep = [[np.ascontiguousarray(a) for a in grp] for grp in (codes, scales, books)]
        sk = [[np.ascontiguousarray(a) for a in sa[k]] for k in ("w", "s", "b")]
        r, w = np.ascontiguousarray(router, np.uint16), np.ascontiguousarray(wsg, np.uint16)
        rc = self.lib.orc_moe_layer_dense_affine_shared(
            C.byref(d), _a(r), _a(w), self._ptrs(keep[0]), self._ptrs(keep[1]), self._ptrs(keep[2]),
            self._ptrs(sk[0]), self._ptrs(sk[1]), self._ptrs(sk[2]), sa["bits"], sa["group"], sa["inter"], sa["fmt"],
            _a(x), M, _a(y), _a(ex), _a(wt), _a(lg), threads)
        assert rc == 0
        return y, ex, wt, lg

    def rmsnorm(self, h, eps=1e-6):
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty_like(h)
        self.lib.orc_rmsnorm(_a(h), h.shape[0], h.shape[1], eps, _a(out))
        return out

    def hc_read(self, desc, w, stream):
        """HyperConnection read: w holds numpy arrays norm, down_w/s/b, up_w/s/b and, with
        injection, inj_w/s/b. Returns (mixed, injection or None, xn, act)."""
        stream = np.ascontiguousarray(stream, np.uint16)
        M = stream.shape[0]
        H, HC, R = desc.hidden, desc.streams, desc.rank
        mixed = np.empty((M, H), np.uint16)
        inj = np.empty((M, HC), np.uint16) if desc.with_injection else None
        xn = np.empty((M, HC * H), np.uint16)
        act = np.empty((M, R), np.float32)
        keep = [np.ascontiguousarray(w[k]) if w.get(k) is not None else None for k in (
            "norm", "down_w", "down_s", "down_b", "up_w", "up_s", "up_b", "inj_w", "inj_s", "inj_b")]
        ptrs = [_a(a) if a is not None else None for a in keep]
        rc = self.lib.orc_hc_read(C.byref(desc), *ptrs, _a(stream), M, _a(mixed),
                                  _a(inj) if inj is not None else None, _a(xn), _a(act))
        assert rc == 0
        return mixed, inj, xn, act

    def hc_write(self, H, HC, stream, block, inj):
        stream = np.ascontiguousarray(stream, np.uint16)
        block = np.ascontiguousarray(block, np.uint16)
        inj = np.ascontiguousarray(inj, np.uint16)
        out = np.empty_like(stream)
        self.lib.orc_hc_write(H, HC, stream.shape[0], _a(stream), _a(block), _a(inj), _a(out))
        return out

    def residual_add(self, h, y):
        h = np.ascontiguousarray(h, np.uint16)
        y = np.ascontiguousarray(y, np.uint16)
        out = np.empty_like(h)
        self.lib.orc_residual_add(_a(h), _a(y), h.size, _a(out))
        return out

    # ---- heads
    def head_q8_synth_logits(self, seed, H, h, v0=0, nv=151936, threads=8):
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty((h.shape[0], nv), np.float32)
        self.lib.orc_head_q8_synth_logits(seed, H, v0, nv, _a(h), h.shape[0], _a(out), threads)
        return out

    def head_q8_logits(self, W, s, h, threads=8):
        W = np.ascontiguousarray(W, np.int8)
        s = np.ascontiguousarray(s, np.uint16)
        h = np.ascontiguousarray(h, np.uint16)
        V, H = W.shape
        out = np.empty((h.shape[0], V), np.float32)
        self.lib.orc_head_q8_logits(_a(W), _a(s), V, H, _a(h), h.shape[0], _a(out), threads)
        return out

    def head_q4_synth_logits(self, seed, H, h, v0=0, nv=151936, threads=8):
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty((h.shape[0], nv), np.float32)
        self.lib.orc_head_q4_synth_logits(seed, H, v0, nv, _a(h), h.shape[0], _a(out), threads)
        return out

    def prepare_u8_book(self, book16, K, D, centered):
        """SparseMoe::prepare_u8_codebook of an FP16 book [K*D] (uint16 bits): (q int32, scales
        fp16 bits [D], biases fp16 bits [D], decoded float values)."""
        b = np.ascontiguousarray(book16, np.uint16)
        q = np.empty(K * D, np.int32)
        s16 = np.empty(D, np.uint16)
        b16 = np.empty(D, np.uint16)
        vals = np.empty(K * D, np.float32)
        self.lib.orc_prepare_u8_book(_a(b), K, D, int(centered), _a(q), _a(s16), _a(b16), _a(vals))
        return q, s16, b16, vals

    def head_q4_logits(self, Wp, s, h, threads=8):
        """Explicit Q4 head: Wp [V, H/2] uint8 (input 2i low nibble, 2i+1 high nibble, signed),
        s [V, H/64] fp16 bits."""
        Wp = np.ascontiguousarray(Wp, np.uint8)
        s = np.ascontiguousarray(s, np.uint16)
        h = np.ascontiguousarray(h, np.uint16)
        V, H = Wp.shape[0], 2 * Wp.shape[1]
        out = np.empty((h.shape[0], V), np.float32)
        self.lib.orc_head_q4_logits(_a(Wp), _a(s), V, H, _a(h), h.shape[0], _a(out), threads)
        return out

    def argmax(self, logits):
        lg = np.ascontiguousarray(logits, np.float32)
        M, V = lg.shape
        idx = np.empty(M, np.uint32)
        val = np.empty(M, np.float32)
        self.lib.orc_argmax(_a(lg), M, V, _a(idx), _a(val))
        return idx, val

    # ---- acceptance
    def decide_greedy(self, drafts, target, stop=()):
        d = np.ascontiguousarray(drafts, np.uint32)
        t = np.ascontiguousarray(target, np.uint32)
        s = np.ascontiguousarray(stop if len(stop) else [0], np.uint32)
        a, r, n = np.zeros(1, np.int64), np.zeros(1, np.int64), np.zeros(1, np.uint32)
        rc = self.lib.orc_decide_greedy(_a(d), len(d), _a(t), len(t), _a(s), len(stop), _a(a), _a(r), _a(n))
        return rc, int(a[0]), int(r[0]), int(n[0])

    def plan_commit(self, off, drafted, accepted):
        out = np.zeros(4, np.uint64)
        rc = self.lib.orc_plan_commit(off, drafted, accepted, _a(out))
        return rc, [int(v) for v in out]

    def philox(self, ctr, key):
        c = np.ascontiguousarray(ctr, np.uint32)
        k = np.ascontiguousarray(key, np.uint32)
        out = np.zeros(4, np.uint32)
        self.lib.orc_philox4x32_10(_a(c), _a(k), _a(out))
        return [int(v) for v in out]

    def round_uniforms(self, seed, slot, rnd, pos):
        u, v = np.zeros(1, np.float32), np.zeros(1, np.float32)
        self.lib.orc_round_uniforms(seed, slot, rnd, pos, _a(u), _a(v))
        return float(u[0]), float(v[0])

    def accept_sampled(self, tl, dl, drafts, T, seed, slot, rnd):
        tl = np.ascontiguousarray(tl, np.float32)
        dl = np.ascontiguousarray(dl, np.float32)
        d = np.ascontiguousarray(drafts, np.uint32)
        a, n = np.zeros(1, np.int64), np.zeros(1, np.uint32)
        rc = self.lib.orc_accept_sampled(_a(tl), _a(dl), _a(d), len(d), tl.shape[1], T, seed, slot, rnd, _a(a), _a(n))
        assert rc == 0
        return int(a[0]), int(n[0])


class RefCore:
    """The reference's own model-free sources compiled by oracle/Makefile (oracle/_ref)."""

    def __init__(self, path=REF_SO):
        self.lib = L = C.CDLL(path)
        sig = lambda n, r, *a: (setattr(getattr(L, n), "restype", r), setattr(getattr(L, n), "argtypes", list(a)))
        sig("ref_packed_vq_word_count", I64, I64, C.c_int)
        sig("ref_unpack_vq_code", C.c_int, P, I64, I64, C.c_int, P)
        sig("ref_supports_segmented_vq", C.c_int, C.c_int, C.c_int)
        sig("ref_decide_greedy", C.c_int, P, I64, P, I64, P, I64, P, P, P)
        sig("ref_plan_commit", C.c_int, U64, U64, U64, P)

    def unpack(self, words, index, bits):
        w = np.ascontiguousarray(words, dtype=np.uint32)
        out = np.zeros(1, np.uint32)
        rc = self.lib.ref_unpack_vq_code(_a(w), len(w), index, bits, _a(out))
        return rc, int(out[0])

    def decide_greedy(self, drafts, target, stop=()):
        d = np.ascontiguousarray(drafts, np.uint32)
        t = np.ascontiguousarray(target, np.uint32)
        s = np.ascontiguousarray(stop if len(stop) else [0], np.uint32)
        a, r, n = np.zeros(1, np.int64), np.zeros(1, np.int64), np.zeros(1, np.uint32)
        rc = self.lib.ref_decide_greedy(_a(d), len(d), _a(t), len(t), _a(s), len(stop), _a(a), _a(r), _a(n))
        return rc, int(a[0]), int(r[0]), int(n[0])

    def plan_commit(self, off, drafted, accepted):
        out = np.zeros(4, np.uint64)
        rc = self.lib.ref_plan_commit(off, drafted, accepted, _a(out))
        return rc, [int(v) for v in out]


_ORACLE = None


def load() -> Oracle:
    global _ORACLE
    if _ORACLE is None:
        _ORACLE = Oracle()
    return _ORACLE


def load_ref():
    return RefCore() if os.path.exists(REF_SO) else None
