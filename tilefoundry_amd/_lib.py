"""ctypes binding of ``libtfdecode_gfx950.so`` (the C ABI in ``include/tf_decode.h``).

There is no fallback: if the library is missing, or was built for an older ABI,
every caller gets a ``RuntimeError`` naming the build command.  A call that
returns non-zero raises ``TFDError`` carrying the library's own message.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_void_p
from functools import lru_cache
from pathlib import Path

from .build import LIB

ABI_VERSION = 16

PRO_PLAIN, PRO_NORM = 0, 1
EPI_STORE, EPI_RESID, EPI_SWIGLU, EPI_LOGITS, EPI_RESID_F32 = 0, 1, 2, 3, 4
ERR_TOKEN_RANGE, ERR_POS_RANGE, ERR_PAGE_RANGE, ERR_STEP_RANGE, ERR_SYNC = 1, 2, 4, 8, 16
ERR_PLACEMENT = 32          # tfd_decode_xcd: a block read an XCC id outside 0..7
PAGE_SIZE = 16
SKINNY_COUNTERS = 16384     # tile counters at the start of a skinny-GEMM work buffer
NOALLOC_SCRATCH_FLOATS = SKINNY_COUNTERS + (1 << 21)   # tfd_gemm_skinny_bf16_noalloc's scratch
ARGMAX_WORK = 128           # int32 per row of tfd_argmax_rows' two-stage work buffer
ATTN_SPLIT = 64
ROUTE_SOFTMAX_TOPK, ROUTE_TOPK_SOFTMAX = 0, 1


def moe_group_words(experts: int, rows: int) -> int:
    """int32 words of tfd_moe_experts' group work buffer (TFD_MOE_GROUP_WORDS)."""
    return 1 + 2 * experts + experts * rows

POLICY_F32, POLICY_BF16 = 0, 1
ROWX_NORM_F32, ROWX_GATED_F32, ROWX_OPERAND, ROWX_ROWS = 0, 1, 2, 3
SMALL_ROWS = 4              # rows of the small-batch entries (tfd_rowgemv_bf16 and the rest)
MOE_ROUTE_GIVEN, MOE_ROUTE_SOFTMAX_TOPK, MOE_ROUTE_TOPK_SOFTMAX = 0, 1, 2


#: tfd_proj8_norm's sizes: rows <= PROJ8_ROWS, K == PROJ8_K
PROJ8_ROWS, PROJ8_K = 8, 4096
#: tfd_sample_rows' limits: top_k <= SAMPLE_MAX_K, vocab <= SAMPLE_MAX_VOCAB
SAMPLE_MAX_K, SAMPLE_MAX_VOCAB = 64, 262144


def moe_packed_fits(rows: int, k: int, hidden: int, inter: int, shared_inter: int) -> bool:
    """Whether tfd_moe_experts_packed takes this shape (its kBadShape check,
    include/tf_hybrid.h): rows <= 16, k <= 16, H a multiple of 1024, I and IS of
    256 with IS <= 2048, rows (k + 1) I / 256 <= 1024."""
    return (rows <= 16 and k <= 16 and hidden % 1024 == 0 and inter % 256 == 0 and
            shared_inter % 256 == 0 and shared_inter <= 2048 and
            rows * (k + 1) * (inter // 256) <= 1024)

P = c_void_p
I = c_int
F = c_float
L = c_int64

#: argtypes of every entry, in header order (restype is int unless named here)
SIGNATURES: dict[str, list] = {
    "tfd_abi_version": [],
    "tfd_last_error": [],
    "tfd_round_bf16": [P, P, I, P],
    "tfd_rmsnorm_bf16": [P, P, P, I, F, P],
    "tfd_embed_bf16": [P, P, P, I, I, P, P],
    "tfd_gemv_bf16": [P, P, P, P, P, I, I, I, I, F, P],
    "tfd_lm_head_argmax_bf16": [P, P, P, P, P, P, I, I, I, F, P],
    "tfd_argmax_finalize": [P, P, I, P, P, P, P, P, I, P, P, I, I, P, P],
    "tfd_attn_rope_scores_paged": [P, P, P, P, P, I, P, P, P, I, P, P, I, I, I, I, F, F, P, I,
                                   P, P, I, P, P],
    "tfd_attn_pv_combine_paged": [P, P, P, I, P, I, I, I, I, P, I, P, P, P, P, I, P, P, P, P],
    "tfd_rmsnorm_rows_bf16": [P, I, P, P, I, I, I, F, I, P],
    "tfd_rmsnorm_rows2_bf16": [P, I, P, P, I, P, I, I, F, P],
    "tfd_pack_skinny_bf16": [P, I, I, I, P, P],
    "tfd_gemm_skinny_bf16": [P, P, I, I, I, I, P, I, P, I, P, L, P],
    "tfd_gemm_skinny_bf16_noalloc": [P, P, I, I, I, I, P, I, P, I, P],
    "tfd_attn_rope_scores_paged_batched": [P, I, P, P, P, P, I, P, P, I, P, P, I, I, I, I, I, F,
                                           F, P, I, P, P, I, I, P, P],
    "tfd_attn_pv_combine_paged_batched": [P, I, P, P, I, P, I, I, I, I, I, P, I, P, P, P, P, I,
                                          I, P, P, P, P],
    "tfd_sample_work_bytes": [I, I, I],
    "tfd_sample_rows": [P, I, I, I, P, P, P, P, L, P],
    "tfd_argmax_rows": [P, I, I, I, P, P, P],
    "tfd_finalize_rows": [P, I, P, I, P, P, P, P, I, I, P, P, I, I, I, P, P],
    "tfd_embed_rows_bf16": [P, P, P, I, I, I, I, P, P],
    "tfd_decode_persistent": [P, I, I, P],
    "tfd_decode_persistent_grid": [],
    "tfd_decode_xcd": [P, P, I, P],
    # include/tf_hybrid.h
    "tfd_pack_skinny_fp8": [P, I, I, I, P, P],
    "tfd_gemm_skinny_fp8": [P, P, P, I, I, I, I, P, I, P, I, P],
    "tfd_gemm_skinny_fp8_resid_scaled": [P, P, P, I, I, I, P, I, F, P, I, P],
    "tfd_route_topk": [P, I, I, I, I, I, P, P, P],
    "tfd_moe_experts": [P, P],
    "tfd_moe_experts_packed": [P, P],
    "tfd_proj8_norm": [P, P],
    "tfd_gdn_step": [P, P],
    "tfd_mamba_step": [P, P],
    "tfd_gqa_decode": [P, P],
    "tfd_rmsnorm_f32_rows": [P, I, P, P, I, P, I, I, F, P],
    "tfd_add_f32_rows": [P, I, P, I, I, I, P],
    "tfd_bf16_to_f32_rows": [P, I, P, I, I, I, P],
    "tfd_scaled_add_rows": [P, I, P, I, I, F, P, I, I, I, P],
    "tfd_tf_rmsnorm_rows_bf16": [P, I, P, P, I, P, I, I, F, P],
    "tfd_gemm_skinny_bf16_logits_div": [P, P, I, I, I, F, P, I, P, L, P],
    "tfd_conv_step_rows": [P, P],
    "tfd_l2norm_f32": [P, P, I, I, F, P],
    "tfd_delta_step_f32": [P, P],
    "tfd_partial_rope_f32": [P, P],
    "tfd_ssm_step_bf16": [P, P],
    "tfd_gated_rmsnorm_bf16": [P, P],
    "tfd_rowgemv_bf16": [P, P],
    "tfd_gdn_step_cols": [P, P, I, P],
    "tfd_moe_experts_small": [P, P],
}
RESTYPES = {"tfd_last_error": ctypes.c_char_p, "tfd_sample_work_bytes": ctypes.c_int64}
UNCHECKED = {"tfd_abi_version", "tfd_decode_persistent_grid"}


class TfdLayer(ctypes.Structure):
    """``TfdLayer`` of include/tf_decode.h (device pointers of one layer)."""

    _fields_ = [(n, c_void_p) for n in ("w_qkv", "w_o", "w_gu", "w_down", "gamma_in",
                                        "gamma_post", "gamma_q", "gamma_k", "k_pool", "v_pool")]


class TfdMoeArgs(ctypes.Structure):
    """``TfdMoeArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [
        *[(n, c_void_p) for n in ("x", "weights", "idx", "w_gate", "w_up", "w_down", "s_gate",
                                   "s_up", "s_down", "w_shared_in", "w_shared_out",
                                   "s_shared_in", "s_shared_out", "w_shared_scale", "hidden",
                                   "shared_scale", "partial", "groups", "out")],
        *[(n, c_int) for n in ("rows", "k", "experts", "hidden_size", "inter", "shared_inter",
                                "hidden_ld", "fp8", "policy", "accumulate")],
        ("logits", c_void_p), ("ldl", c_int), ("route", c_int),
        ("err", c_void_p), ("resid", c_void_p), ("resid_mult", c_float),
    ]


class TfdSampling(ctypes.Structure):
    """include/tf_decode.h TfdSampling (tfd_sample_rows): top_k 0 samples the whole
    row by Gumbel-max, 1..SAMPLE_MAX_K the top k with the top_p nucleus."""
    _fields_ = [("temperature", c_float), ("top_k", c_int), ("top_p", c_float),
                ("seed", ctypes.c_uint64)]


class TfdProj8NormArgs(ctypes.Structure):
    """``TfdProj8NormArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [
        ("x", c_void_p), ("ldx", c_int), ("gamma", c_void_p), ("eps", c_float),
        ("x_rows", c_void_p), ("ldxr", c_int), ("w", c_void_p), ("scale", c_void_p),
        *[(n, c_int) for n in ("rows", "K", "N")],
        ("out", c_void_p), ("ldo", c_int), ("epilogue", c_int),
    ]


class TfdGdnArgs(ctypes.Structure):
    """``TfdGdnArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [
        ("proj", c_void_p), ("proj_ld", c_int),
        *[(n, c_void_p) for n in ("conv_in", "conv_out", "state", "conv_w", "a_log", "dt_bias",
                                   "gamma", "out")],
        *[(n, c_int) for n in ("rows", "key_heads", "value_heads", "head_k_dim", "head_v_dim",
                                "conv_kernel")],
        ("l2_eps", c_float), ("rms_eps", c_float),
    ]


class TfdMambaArgs(ctypes.Structure):
    """``TfdMambaArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [
        ("proj", c_void_p), ("proj_ld", c_int),
        *[(n, c_void_p) for n in ("conv_in", "conv_out", "state", "conv_w", "conv_b", "a_log",
                                   "dt_bias", "d_skip", "gamma", "gated", "ssq", "out")],
        *[(n, c_int) for n in ("rows", "heads", "head_dim", "state_dim", "groups",
                                "conv_kernel")],
        ("eps", c_float),
    ]


class TfdGqaArgs(ctypes.Structure):
    """``TfdGqaArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [
        ("qkv", c_void_p), ("ldq", c_int),
        *[(n, c_void_p) for n in ("gamma_q", "gamma_k", "cos_table", "sin_table")],
        ("rope_rows", c_int), ("rot_dim", c_int),
        ("pos", c_void_p), ("page_table", c_void_p), ("max_pages", c_int),
        ("k_pool", c_void_p), ("v_pool", c_void_p), ("num_pages", c_int),
        *[(n, c_int) for n in ("rows", "heads", "kv_heads", "head_dim")],
        ("scale", c_float), ("eps", c_float),
        ("scores", c_void_p), ("score_stride", c_int),
        ("stats", c_void_p), ("part", c_void_p), ("counters", c_void_p),
        ("nsplit", c_int), ("split_len", c_int),
        ("out", c_void_p), ("policy", c_int), ("err", c_void_p),
    ]


class TfdConvStepArgs(ctypes.Structure):
    """``TfdConvStepArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [("window", c_void_p), ("entry", c_void_p), ("lde", c_int),
                ("conv_w", c_void_p), ("conv_b", c_void_p), ("out", c_void_p),
                *[(n, c_int) for n in ("ldo", "rows", "channels", "kernel", "policy")]]


class TfdDeltaStepArgs(ctypes.Structure):
    """``TfdDeltaStepArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [*[(n, c_void_p) for n in ("state_in", "state_out", "q", "k", "v", "g", "beta",
                                           "read")],
                ("qscale", c_float),
                *[(n, c_int) for n in ("rows", "heads", "head_k_dim", "head_v_dim")]]


class TfdPartialRopeArgs(ctypes.Structure):
    """``TfdPartialRopeArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [("x", c_void_p), ("ldx", c_int), ("out", c_void_p), ("ldo", c_int),
                ("pos", c_void_p), ("cos_table", c_void_p), ("sin_table", c_void_p),
                *[(n, c_int) for n in ("rope_rows", "rows", "heads", "head_dim", "rot")]]


class TfdSsmStepArgs(ctypes.Structure):
    """``TfdSsmStepArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [("state_in", c_void_p), ("state_out", c_void_p), ("x", c_void_p), ("ldx", c_int),
                ("b_vec", c_void_p), ("ldb", c_int), ("c_vec", c_void_p), ("ldc", c_int),
                ("dt_raw", c_void_p), ("lddt", c_int),
                *[(n, c_void_p) for n in ("a_log", "dt_bias", "d_skip", "y")],
                *[(n, c_int) for n in ("ldy", "rows", "heads", "head_dim", "state_dim")]]


class TfdGatedNormArgs(ctypes.Structure):
    """``TfdGatedNormArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [("y", c_void_p), ("ldy", c_int), ("gate", c_void_p), ("ldg", c_int),
                ("gamma", c_void_p), ("out", c_void_p),
                *[(n, c_int) for n in ("ldo", "rows", "n")], ("eps", c_float)]


class TfdRowGemvArgs(ctypes.Structure):
    """``TfdRowGemvArgs`` of include/tf_hybrid.h, field for field."""

    _fields_ = [("x", c_void_p), ("ldx", c_int), ("x_kind", c_int), ("gamma", c_void_p),
                ("gate", c_void_p), ("ldg", c_int), ("head_dim", c_int), ("eps", c_float),
                ("w", c_void_p), ("K", c_int), ("N", c_int), ("out", c_void_p), ("ldo", c_int),
                ("epilogue", c_int), ("x_rows", c_void_p), ("ldxr", c_int), ("rows", c_int)]


class TfdDecodeArgs(ctypes.Structure):
    """``TfdDecodeArgs`` of include/tf_decode.h, field for field."""

    _fields_ = [
        ("layers", c_void_p),
        *[(n, c_int) for n in ("n_layers", "hidden", "heads", "kv_heads", "head_dim",
                                "intermediate", "vocab")],
        ("eps", c_float), ("scale", c_float),
        *[(n, c_void_p) for n in ("w_embed", "w_head", "gamma_final", "cos_table",
                                   "sin_table")],
        ("rope_rows", c_int),
        ("page_table", c_void_p),
        ("max_pages", c_int), ("num_pages", c_int),
        *[(n, c_void_p) for n in ("x_hid", "x_h1", "x_qkv", "x_attn", "x_mid", "x_smax",
                                   "x_psum", "x_pout", "x_best")],
        ("epoch", ctypes.c_uint32),
        ("scores", c_void_p), ("score_stride", c_int),
        ("score_new", c_void_p),
        ("nsplit", c_int),
        *[(n, c_void_p) for n in ("logits", "ids", "pos", "inp", "prompt_len", "sam")],
        ("nsteps", c_int),
        ("err", c_void_p),
        ("timeline", c_void_p), ("timeline_steps", c_int),
    ]


class TfdXcdArgs(ctypes.Structure):
    """``TfdXcdArgs`` of include/tf_decode.h (the XCD-partitioned kernel's arenas)."""

    _fields_ = [(n, c_void_p) for n in ("hid", "h1", "opart", "dpart", "smax", "psum", "pout")]


XCDS = 8                    # XCDs of an MI355X, the unit of tfd_decode_xcd's partition


def timeline_stamps(n_layers: int) -> int:
    """Stamps per step of the persistent kernel's timeline (TFD_TIMELINE_STAMPS)."""
    return 14 * n_layers + 4


def tags_per_step(n_layers: int) -> int:
    """Flag-in-data tags one persistent step uses (TFD_TAGS_PER_STEP)."""
    return n_layers + 1


class TFDError(RuntimeError):
    """A library entry rejected its arguments or failed to launch."""

    def __init__(self, name: str, code: int, message: str):
        super().__init__(f"{name} returned {code}: {message}")
        self.code = code


class _Checked:
    """Wraps the CDLL so every int-returning entry raises on a non-zero result."""

    def __init__(self, dll: ctypes.CDLL):
        self._dll = dll
        for name, args in SIGNATURES.items():
            fn = getattr(dll, name)
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, ctypes.c_int)

    def last_error(self) -> str:
        return self._dll.tfd_last_error().decode(errors="replace")

    def __getattr__(self, name):
        fn = getattr(self._dll, name)
        if name in RESTYPES or name in UNCHECKED:
            return fn

        def call(*args):
            rc = fn(*args)
            if rc != 0:
                raise TFDError(name, rc, self.last_error())
            return rc

        return call


@lru_cache(maxsize=1)
def lib() -> _Checked:
    """The loaded library (loaded once per process)."""
    path = Path(LIB)
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built: run `python -m tilefoundry_amd.build` "
            "(or __graft_entry__.build()) first; there is no non-HIP fallback")
    dll = ctypes.CDLL(str(path))
    got = dll.tfd_abi_version()
    if got != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI {got}, this package expects {ABI_VERSION}: rebuild it")
    return _Checked(dll)


def ptr(t) -> int:
    """Device address of a torch tensor (0 for None)."""
    return 0 if t is None else t.data_ptr()
