"""ctypes binding of libq38.so (include/q38.h), the C ABI of the gfx950 verify round.

This module is plumbing for tests and the benchmark: it loads the in-tree shared library
and exposes the ABI's structs and functions. It has no fallback: if libq38.so is missing
or fails to load, importing it raises.

libq38.so links libamdhip64 by soname. A PyTorch build for ROCm carries its own copy: when
both are used in one process, import torch first, so that the library binds to the runtime
torch already loaded and the process holds a single HIP runtime.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# (Q38_LIB: another build of the same ABI, e.g. the phase-stamp build trace/libq38.so)
LIB_PATH = os.environ.get("Q38_LIB") or os.path.join(_HERE, "libq38.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"libq38.so is not built at {LIB_PATH}; run __graft_entry__.build()")
lib = C.CDLL(LIB_PATH)

Q38_OK, Q38_EINVAL, Q38_ERANGE, Q38_EHIP, Q38_ENOMEM, Q38_ESTATE, Q38_ESPACE, Q38_EWAIT = 0, -1, -2, -3, -4, -5, -6, -7
Q38_HEAD_Q8, Q38_HEAD_Q4G64 = 0, 1
Q38_CB_FP16, Q38_CB_INT8_SCALED, Q38_CB_U8_PERDIM = 0, 1, 2


class Q38Error(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"q38 error {code}: {msg}")
        self.code = code


class MoeDesc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "hidden", "inter", "experts", "top_k", "gu_dim", "gu_bits", "down_dim", "down_bits",
        "gu_group", "down_group", "normalize_topk", "has_shared", "mixed", "book_format")]


class MoeWeights(C.Structure):
    _fields_ = [("router", C.c_void_p), ("shared_gate", C.c_void_p),
                ("codes", C.c_void_p * 3), ("scales", C.c_void_p * 3), ("books", C.c_void_p * 3)]


class MoeMixedWeights(C.Structure):
    _fields_ = [("router", C.c_void_p), ("shared_gate", C.c_void_p), ("codes_d4", C.c_void_p * 3),
                ("scales_d4", C.c_void_p * 3), ("books_d4", C.c_void_p * 3), ("codes_d8", C.c_void_p * 3),
                ("scales_d8", C.c_void_p * 3), ("books_d8", C.c_void_p * 3), ("book_scales_d8", C.c_uint16 * 3),
                ("reserved", C.c_uint16)]


class GdnDesc(C.Structure):  # include/q38.h q38_gdn_desc
    _fields_ = [(n, C.c_int32) for n in ("hidden", "key_heads", "value_heads", "key_dim", "value_dim", "conv_kernel",
                                         "bits", "group", "scale_dtype", "gate_silu")] + [("eps", C.c_float)]


class GdnWeights(C.Structure):  # include/q38.h q38_gdn_weights
    _fields_ = [("weight", C.c_void_p * 5), ("scales", C.c_void_p * 5), ("biases", C.c_void_p * 5),
                ("conv", C.c_void_p), ("a_log", C.c_void_p), ("dt_bias", C.c_void_p), ("norm", C.c_void_p)]


class AttnDesc(C.Structure):  # include/q38.h q38_attn_desc
    _fields_ = [(n, C.c_int32) for n in ("hidden", "q_heads", "kv_heads", "head_dim", "rotary_dim", "bits", "group",
                                         "scale_dtype", "norm_offset")] + [("eps", C.c_float),
                                                                            ("rope_theta", C.c_double)]


class AttnWeights(C.Structure):  # include/q38.h q38_attn_weights
    _fields_ = [("weight", C.c_void_p * 4), ("scales", C.c_void_p * 4), ("biases", C.c_void_p * 4),
                ("q_norm", C.c_void_p), ("k_norm", C.c_void_p)]


class AffineShared(C.Structure):
    _fields_ = [("weight", C.c_void_p * 3), ("scales", C.c_void_p * 3), ("biases", C.c_void_p * 3),
                ("bits", C.c_int32), ("group", C.c_int32), ("inter", C.c_int32), ("scale_dtype", C.c_int32)]


class RouteOut(C.Structure):
    _fields_ = [("experts", C.c_void_p), ("weights", C.c_void_p), ("logits", C.c_void_p),
                ("plan", C.c_void_p), ("x_norm", C.c_void_p)]


class MoeTimings(C.Structure):
    _fields_ = [("routing_ms", C.c_double), ("gate_up_ms", C.c_double), ("down_ms", C.c_double),
                ("merge_ms", C.c_double), ("layers", C.c_int32), ("reserved", C.c_int32)]


class GreedyDecision(C.Structure):
    _fields_ = [("accepted", C.c_int64), ("correction_row", C.c_int64), ("next_token", C.c_uint32)]


def _sig(name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


P, I32, I64, U32, U64, SZ, F32 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_size_t, C.c_float
_sig("q38_last_error", C.c_char_p)
_sig("q38_version", C.c_char_p)
_sig("q38_ctx_create", C.c_int, C.c_int, C.POINTER(P))
_sig("q38_ctx_destroy", None, P)
_sig("q38_ctx_synchronize", C.c_int, P, P)
_sig("q38_set_fused_layers", None, C.c_int)
_sig("q38_set_u8_native", None, C.c_int)
_sig("q38_debug_set_wait_limit", None, I32)
_sig("q38_gdn_create", C.c_int, P, C.POINTER(GdnDesc), C.POINTER(GdnWeights), C.POINTER(P))
_sig("q38_gdn_destroy", None, P)
_sig("q38_gdn_state_bytes", C.c_size_t, P)
_sig("q38_gdn_workspace_size", C.c_size_t, P, I32)
_sig("q38_gdn_verify", C.c_int, P, P, I32, P, P, P, P, C.c_size_t, P)
_sig("q38_gdn_commit", C.c_int, P, P, I32, P, P)
_sig("q38_attn_create", C.c_int, P, C.POINTER(AttnDesc), C.POINTER(AttnWeights), C.POINTER(P))
_sig("q38_attn_destroy", None, P)
_sig("q38_attn_cache_bytes", C.c_size_t, P, I64)
_sig("q38_attn_workspace_size", C.c_size_t, P, I32, I64)
_sig("q38_attn_verify", C.c_int, P, P, I32, P, I64, I64, I64, P, P, C.c_size_t, P)
_sig("q38_packed_vq_word_count", I64, I64, C.c_int)
_sig("q38_unpack_vq_code", C.c_int, P, I64, I64, C.c_int, C.POINTER(U32))
_sig("q38_supports_segmented_vq", C.c_int, C.c_int, C.c_int)
_sig("q38_moe_layer_create", C.c_int, P, C.POINTER(MoeDesc), C.POINTER(MoeWeights), C.POINTER(P))
_sig("q38_moe_layer_create_synthetic", C.c_int, P, C.POINTER(MoeDesc), U64, I32, C.POINTER(P))
_sig("q38_moe_layer_create_affine_shared", C.c_int, P, C.POINTER(MoeDesc), C.POINTER(MoeWeights),
     C.POINTER(AffineShared), C.POINTER(P))
_sig("q38_moe_layer_destroy", None, P)
_sig("q38_moe_layer_load", C.c_int, P, C.c_char_p, C.c_char_p, I32, C.POINTER(P))
_sig("q38_checkpoint_inspect", C.c_int, C.c_char_p, C.c_char_p, C.POINTER(MoeDesc))
_sig("q38_moe_layer_weights", C.c_int, P, C.POINTER(MoeWeights))
_sig("q38_moe_layer_mixed_weights", C.c_int, P, C.POINTER(MoeMixedWeights))
_sig("q38_moe_layer_create_mixed", C.c_int, P, C.POINTER(MoeDesc), C.POINTER(MoeMixedWeights), C.POINTER(P))
_sig("q38_moe_layer_codebook", C.c_int, P, C.c_int, C.POINTER(P), C.POINTER(P), C.POINTER(P), C.POINTER(P))
_sig("q38_moe_layer_bytes", I64, P, I32, I32)
_sig("q38_moe_workspace_size", SZ, C.POINTER(MoeDesc), I32)
_sig("q38_moe_route", C.c_int, P, P, I32, C.POINTER(RouteOut), P, SZ, P)
_sig("q38_moe_forward", C.c_int, P, P, I32, P, C.POINTER(RouteOut), P, SZ, P)
_sig("q38_moe_forward_static", C.c_int, P, P, I32, P, C.POINTER(RouteOut), P)
_sig("q38_moe_forward_prefill_profiled", C.c_int, P, P, I32, P, C.POINTER(RouteOut), P, SZ, C.POINTER(F32), P)
_sig("q38_moe_layer_set_router_bias", C.c_int, P, P)
_sig("q38_verify_chain", C.c_int, C.POINTER(P), I32, P, I32, F32, C.POINTER(RouteOut), P, SZ, P)
_sig("q38_verify_chain_profiled", C.c_int, C.POINTER(P), I32, P, I32, F32, C.POINTER(RouteOut), P, SZ,
     C.POINTER(MoeTimings), P)
_sig("q38_rmsnorm", C.c_int, P, I32, I32, F32, P, P)
_sig("q38_embed_synthetic", C.c_int, U64, C.POINTER(U32), I32, I32, P, P)
_sig("q38_embed_synthetic_dev", C.c_int, U64, P, I32, I32, P, P)
_sig("q38_head_create", C.c_int, P, C.c_int, I64, I32, P, P, C.POINTER(P))
_sig("q38_head_create_synthetic", C.c_int, P, C.c_int, I64, I32, U64, C.POINTER(P))
_sig("q38_head_destroy", None, P)
_sig("q38_head_weights", C.c_int, P, C.POINTER(P), C.POINTER(P))
_sig("q38_head_bytes", I64, P)
_sig("q38_head_workspace_size", SZ, P, I32)
_sig("q38_head_greedy", C.c_int, P, P, I32, P, P, P, SZ, P)
_sig("q38_head_logits", C.c_int, P, P, I32, P, P, SZ, P)
_sig("q38_head_probs_workspace_size", SZ, P, I32)
_sig("q38_head_probs", C.c_int, P, P, I32, C.c_float, P, P, P, SZ, P)
_sig("q38_argmax_rows", C.c_int, P, I32, I64, P, P, P, SZ, P)


class MtpTrace(C.Structure):
    _fields_ = [("combined", P), ("final_mixed", P)]


Q38_MTP_FC_EMBED_SALT = 0x46C0E3BE
Q38_MTP_FC_HIDDEN_SALT = 0x46C0411D
_sig("q38_mtp_head_create", C.c_int, P, P, P, P, P, U64, F32, C.POINTER(P))
_sig("q38_mtp_head_create_synthetic", C.c_int, P, C.POINTER(MoeDesc), I64, U64, C.POINTER(P))
_sig("q38_mtp_head_destroy", None, P)
_sig("q38_mtp_head_parts", C.c_int, P, C.POINTER(P), C.POINTER(P), C.POINTER(P), C.POINTER(P))
_sig("q38_mtp_workspace_size", SZ, P, I32)
_sig("q38_mtp_forward_decode", C.c_int, P, P, P, I32, P, P, C.POINTER(MtpTrace), P, SZ, P)
_sig("q38_mtp_draft_greedy", C.c_int, P, P, P, I32, I32, P, P, P, SZ, P)
_sig("q38_mtp_decide_greedy", C.c_int, C.POINTER(U32), I64, C.POINTER(U32), I64, C.POINTER(U32), I64,
     C.POINTER(GreedyDecision))
_sig("q38_plan_mtp_commit", C.c_int, U64, U64, U64, C.POINTER(U64))
_sig("q38_mtp_accept_sampled", C.c_int, P, P, P, I32, I64, F32, U64, U64, U64, P, P, SZ, P)
_sig("q38_mtp_accept_workspace_size", SZ, I32, I64)
_sig("q38_philox4x32_10", None, C.POINTER(U32), C.POINTER(U32), C.POINTER(U32))
_sig("q38_slot_create", C.c_int, P, I32, I32, U64, C.POINTER(P))
_sig("q38_slot_destroy", None, P)
_sig("q38_slot_stage", C.c_int, P, I32, P, P)
_sig("q38_slot_commit", C.c_int, P, I64, P)
_sig("q38_slot_rollback", C.c_int, P)
_sig("q38_slot_info", C.c_int, P, C.POINTER(U64), C.POINTER(I32), C.POINTER(I32))
_sig("q38_slot_hidden", P, P)
_sig("q38_slot_generation", C.c_uint64, P)


class HcDesc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("hidden", "streams", "rank", "bits", "group", "with_injection")] + [
        ("eps", C.c_float)]


class HcWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "norm", "down_w", "down_s", "down_b", "up_w", "up_s", "up_b", "inj_w", "inj_s", "inj_b")]


_sig("q38_hc_create", C.c_int, P, C.POINTER(HcDesc), C.POINTER(HcWeights), C.POINTER(P))
_sig("q38_hc_destroy", None, P)
_sig("q38_hc_workspace_size", SZ, C.POINTER(HcDesc), I32)
_sig("q38_hc_read", C.c_int, P, P, I32, P, P, P, SZ, P)
_sig("q38_hc_write", C.c_int, P, P, P, P, I32, P, P)
_sig("q38_hc_initialize_stream", C.c_int, P, I32, I32, I32, P, P)


class MlpMap(C.Structure):  # include/q38.h q38_mlp_map
    _fields_ = [("hidden", C.c_int32), ("rank", C.c_int32), ("full", C.c_void_p), ("left", C.c_void_p),
                ("right", C.c_void_p)]


_sig("q38_mlp_map_workspace_size", SZ, C.POINTER(MlpMap), I32)
_sig("q38_mlp_output_map", C.c_int, C.POINTER(MlpMap), P, I32, P, P, SZ, P)
_sig("q38_verify_chain_hc_mapped_workspace_size", SZ, C.POINTER(MoeDesc), C.POINTER(HcDesc), I32)
_sig("q38_verify_chain_hc_mapped", C.c_int, C.POINTER(P), C.POINTER(P), C.POINTER(C.POINTER(MlpMap)), I32, P, I32, P,
     SZ, P)


class MtpStreams(C.Structure):
    _fields_ = [("block_mixer", P), ("final_mixer", P), ("embedding_norm", P), ("hidden_norm", P)]


_sig("q38_mtp_head_set_streams", C.c_int, P, C.POINTER(MtpStreams))
_sig("q38_mtp_head_streams", C.c_int, P)
_sig("q38_verify_chain_hc_workspace_size", SZ, C.POINTER(MoeDesc), C.POINTER(HcDesc), I32)
_sig("q38_verify_chain_hc", C.c_int, P, P, I32, P, I32, P, SZ, P)


def check(rc: int) -> int:
    if rc != Q38_OK:
        raise Q38Error(rc, lib.q38_last_error().decode())
    return rc


def last_error() -> str:
    return lib.q38_last_error().decode()


def desc(hidden=2048, inter=512, experts=512, top_k=10, gu=(8, 14), down=(8, 14), gu_group=None,
         down_group=None, normalize=1, shared=1, mixed=0, book_format=0) -> MoeDesc:
    """Layer description; groups default to one scale per output row."""
    return MoeDesc(hidden, inter, experts, top_k, gu[0], gu[1], down[0], down[1],
                   gu_group or hidden, down_group or inter, normalize, shared, mixed, book_format)


def words_per_row(n_in: int, dim: int, bits: int) -> int:
    return ((n_in // dim + 31) // 32) * bits


def ptr(t) -> int:
    """Device/host address of a torch tensor (or an int address)."""
    return t if isinstance(t, int) else t.data_ptr()


class Ctx:
    def __init__(self, device: int = 0):
        h = P()
        check(lib.q38_ctx_create(device, C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib.q38_ctx_destroy(self.h)
            self.h = None


class MoeLayer:
    def __init__(self, ctx: Ctx, d: MoeDesc, seed: int | None = None, layer: int = 0,
                 weights: MoeWeights | None = None):
        h = P()
        self.desc = d
        if weights is None:
            check(lib.q38_moe_layer_create_synthetic(ctx.h, C.byref(d), seed, layer, C.byref(h)))
        else:
            check(lib.q38_moe_layer_create(ctx.h, C.byref(d), C.byref(weights), C.byref(h)))
        self.h = h

    def weights(self) -> MoeWeights:
        w = MoeWeights()
        check(lib.q38_moe_layer_weights(self.h, C.byref(w)))
        return w

    def codebook(self, proj: int):
        """Device pointers (book, q, scales, biases) of the codebook the kernels read."""
        ptrs = [P() for _ in range(4)]
        check(lib.q38_moe_layer_codebook(self.h, proj, *[C.byref(x) for x in ptrs]))
        return [x.value for x in ptrs]

    def bytes(self, n_unique: int, rows: int) -> int:
        return lib.q38_moe_layer_bytes(self.h, n_unique, rows)

    def close(self):
        if self.h:
            lib.q38_moe_layer_destroy(self.h)
            self.h = None


class Head:
    def __init__(self, ctx: Ctx, kind: int, vocab: int, hidden: int, seed: int | None = None,
                 weights=None, scales=None):
        h = P()
        if weights is None:
            check(lib.q38_head_create_synthetic(ctx.h, kind, vocab, hidden, seed, C.byref(h)))
        else:
            check(lib.q38_head_create(ctx.h, kind, vocab, hidden, ptr(weights), ptr(scales), C.byref(h)))
        self.h, self.kind, self.vocab, self.hidden = h, kind, vocab, hidden

    def workspace_size(self, rows: int) -> int:
        return lib.q38_head_workspace_size(self.h, rows)

    def device_weights(self):
        w, s = P(), P()
        check(lib.q38_head_weights(self.h, C.byref(w), C.byref(s)))
        return w.value, s.value

    def close(self):
        if self.h:
            lib.q38_head_destroy(self.h)
            self.h = None


class MtpHead:
    """The MTP draft head (q38_mtp_head): synthetic (seeded) with the given MoE geometry."""

    def __init__(self, ctx: Ctx, d: MoeDesc, vocab: int, seed: int):
        h = P()
        check(lib.q38_mtp_head_create_synthetic(ctx.h, C.byref(d), vocab, seed, C.byref(h)))
        self.h, self.desc, self.vocab, self.seed = h, d, vocab, seed

    def workspace_size(self, rows: int) -> int:
        return lib.q38_mtp_workspace_size(self.h, rows)

    def set_streams(self, block: "Hc", final: "Hc", embedding_norm=None, hidden_norm=None):
        """Run the head on HC streams (q38_mtp_head_set_streams); the mixers and norm tensors
        must outlive the head's use of them."""
        self._streams = (block, final, embedding_norm, hidden_norm)
        s = MtpStreams(block.h, final.h, None if embedding_norm is None else ptr(embedding_norm),
                       None if hidden_norm is None else ptr(hidden_norm))
        check(lib.q38_mtp_head_set_streams(self.h, C.byref(s)))

    def clear_streams(self):
        check(lib.q38_mtp_head_set_streams(self.h, None))
        self._streams = None

    def parts(self):
        layer, fe, fh, dh = P(), P(), P(), P()
        check(lib.q38_mtp_head_parts(self.h, C.byref(layer), C.byref(fe), C.byref(fh), C.byref(dh)))
        return layer.value, fe.value, fh.value, dh.value

    def close(self):
        if self.h:
            lib.q38_mtp_head_destroy(self.h)
            self.h = None


def routes(experts=None, weights=None, logits=None, plan=None, x_norm=None) -> RouteOut:
    f = lambda t: None if t is None else ptr(t)
    return RouteOut(f(experts), f(weights), f(logits), f(plan), f(x_norm))


class Hc:
    """HyperConnection mixer over caller-owned device weights (torch tensors keyed by the
    q38_hc_weights field names; the handle keeps references to them)."""

    _FIELDS = ("norm", "down_w", "down_s", "down_b", "up_w", "up_s", "up_b", "inj_w", "inj_s", "inj_b")

    def __init__(self, ctx: "Ctx", desc: HcDesc, tensors: dict):
        self.desc = desc
        self._keep = tensors
        w = HcWeights(*[ptr(tensors[k]) if tensors.get(k) is not None else None for k in self._FIELDS])
        h = P()
        check(lib.q38_hc_create(ctx.h, C.byref(desc), C.byref(w), C.byref(h)))
        self.h = h

    def workspace_size(self, rows: int) -> int:
        return lib.q38_hc_workspace_size(C.byref(self.desc), rows)

    def read(self, stream, rows, mixed, injection, ws, st=None):
        check(lib.q38_hc_read(self.h, ptr(stream), rows, ptr(mixed), ptr(injection) if injection is not None else None,
                              ptr(ws), ws.numel() if hasattr(ws, "numel") else 0, st))

    def write(self, stream, block, injection, rows, out, st=None):
        check(lib.q38_hc_write(self.h, ptr(stream), ptr(block), ptr(injection), rows, ptr(out), st))

    def close(self):
        if self.h:
            lib.q38_hc_destroy(self.h)
            self.h = None
