"""The hot-path op kinds with their gfx950 bindings (names as in ``monolith/ops/{gemv,norm,attention,gdn,moe}.py``).

``gdn_commit`` (the speculative verify's state commit, ``ops/gdn.py:13-17``) is the GDN step entry point with
``commit = 1``: the committed tokens replayed from the step's input slot into its output slot, no read-out."""

from .registry import PROFILE, KernelBinding, OpClass, OpDef, register_op


def _op(name, klass, domain, kernel=None, **consts):
    od = OpDef(name, klass, domain)
    if kernel is not None:
        od.bind(PROFILE, KernelBinding(kernel, dict(consts)))
    return register_op(od)


GEMV = _op("gemv", OpClass.MAP, "rows", "mi_gemv")
LM_HEAD = _op("lm_head", OpClass.MAP, "rows", "mi_gemv", out_f32=1)
# standalone kernels; a norm that feeds a GEMV is fused into its load instead (mi_gemv_desc.norm_w)
RMSNORM_STAT = _op("rmsnorm_stat", OpClass.REDUCE, "span", "mi_rmsnorm_stat")
NORM_APPLY = _op("norm_apply", OpClass.MAP, "span", "mi_norm_apply")
GQA_DECODE = _op("gqa_decode", OpClass.MAP, "heads", "mi_gqa_decode")
GQA_MERGE = _op("gqa_merge", OpClass.MAP, "heads", "mi_gqa_decode", fused_into="gqa_decode")
GDN_MIXER = _op("gdn_mixer", OpClass.MAP, "heads", "mi_gdn_step")
GDN_NORM = _op("gdn_norm", OpClass.MAP, "heads", "mi_gdn_step", fused_into="gdn_mixer")
GDN_COMMIT = _op("gdn_commit", OpClass.MAP, "heads", "mi_gdn_step", commit=1)
MOE_ROUTE = _op("moe_route", OpClass.MAP, "rows", "mi_moe_route")
MOE_GEMV = _op("moe_gemv", OpClass.MAP, "rows", "mi_gemv", grouped=1)
MOE_COMBINE = _op("moe_combine", OpClass.MAP, "rows", "mi_moe_combine")
EMBED = _op("embed", OpClass.MAP, "rows", "mi_embed")                       # ops/embed.py:1-7
ARGMAX = _op("argmax", OpClass.REDUCE, "span", "mi_argmax")                 # ops/sample.py:9
SAMPLE = _op("sample", OpClass.REDUCE, "span", "mi_sample")                 # ops/sample.py:10
VERIFY_SELECT = _op("verify_select", OpClass.SERIAL, "span", "mi_verify_select")   # ops/draft.py:27
ACCEPT_SCAN = _op("accept_scan", OpClass.SERIAL, "span", "mi_accept_scan")         # ops/draft.py:28

DECODE_LAYER_OPS = ("gemv", "rmsnorm_stat", "norm_apply", "gqa_decode", "gqa_merge", "gdn_mixer", "gdn_norm",
                    "gdn_commit", "moe_route", "moe_gemv", "moe_combine", "lm_head")

# the token loop around the layers; the program's tail (the advance, compiler/emit.py:1459-1462) is mi_advance
STEP_OPS = ("embed", "argmax", "sample", "verify_select", "accept_scan")
