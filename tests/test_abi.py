"""The C-ABI boundary: the library loads without a GPU and exports every
function include/*.h declares (no compute calls here)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")


def declared_functions():
    names = set()
    for fn in os.listdir(INC):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INC, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(qwen_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("qwen_hip_decoder_create", "qwen_hip_decoder_prefill", "qwen_hip_decoder_forward",
                 "qwen_hip_decoder_generate", "qwen_hip_decoder_set_kv_len", "qwen_hip_linear_nobias_bf16",
                 "qwen_hip_causal_attention", "qwen_hip_argmax_matvec_bf16", "qwen_hip_rms_norm"):
        assert must in names


def test_library_exports_every_declared_symbol(qa):
    lib = qa.lib()
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing
    # and the ctypes view binds exactly the declared set
    assert {s[0] for s in qa.SIGNATURES} == declared_functions()


def test_host_only_calls_work_without_gpu(qa):
    c = qa.preset(0)
    assert (c.hidden, c.layers, c.heads, c.kv_heads, c.head_dim, c.intermediate, c.vocab) == \
        (1024, 28, 16, 8, 128, 3072, 151936)
    c = qa.preset(1)
    assert (c.hidden, c.intermediate) == (2048, 6144)
    assert qa.lib().qwen_f32_to_bf16_rne(1.0) == 0x3F80
