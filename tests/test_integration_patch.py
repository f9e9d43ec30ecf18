"""The integration patch (integration/mlxcel-libmlxq.patch) that routes the
reference's ROCm QuantizedMatmul / GatherQMM / dequantize evals to libmlxq
applies cleanly to the reference's own files, and after applying it every
hook sits in its eval_gpu ahead of the backend's kernels.  The patch is
checked against scratch copies of the files it changes (the reference tree
is read, never written).  Skipped where the reference is absent (the GPU
box)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATCH = os.path.join(ROOT, "integration", "mlxcel-libmlxq.patch")
REF = "/root/reference"


def patched_files():
    text = open(PATCH).read()
    old = re.findall(r"^--- a/(\S+)$", text, re.M)
    new = re.findall(r"^\+\+\+ b/(\S+)$", text, re.M)
    return old, new


@pytest.mark.skipif(not os.path.isdir(REF), reason="the reference tree is not present here")
def test_patch_applies_to_the_reference_files(tmp_path):
    old, new = patched_files()
    assert old, "the patch changes no existing file"
    for rel in old:
        dst = tmp_path / rel
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copyfile(os.path.join(REF, rel), dst)
    subprocess.run(["git", "init", "-q"], cwd=tmp_path, check=True)
    r = subprocess.run(["git", "apply", "--check", "-v", PATCH], cwd=tmp_path, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run(["git", "apply", PATCH], cwd=tmp_path, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    for rel in new:
        assert (tmp_path / rel).exists(), rel
    qmm = next(p for p in old if p.endswith("quantized/qmm.hip"))
    src = (tmp_path / qmm).read_text()
    for fn, hook in (("QuantizedMatmul::eval_gpu", "rocm::mlxq_quantized_matmul("),
                     ("GatherQMM::eval_gpu", "rocm::mlxq_gather_qmm(")):
        body = src[src.index("void " + fn):]
        # the hook comes right after the output allocation, before the first kernel setup
        assert body.index(hook) < body.index("ensure_row_contiguous_matrix"), fn
    qcpp = next(p for p in old if p.endswith("quantized/quantized.cpp"))
    src = (tmp_path / qcpp).read_text()
    body = src[src.index("void fast::Quantize::eval_gpu"):]
    assert body.index("rocm::mlxq_dequantize(") < body.index("affine_dequantize(wq")


def test_patch_declares_the_abi_it_calls():
    # the hooks call libmlxq through dlsym: each symbol they resolve is one
    # include/mlxq.h declares, with the same argument count
    text = open(PATCH).read()
    header = open(os.path.join(ROOT, "include", "mlxq.h")).read()
    syms = re.findall(r'dlsym\(h, "(mlxq_\w+)"\)', text)
    assert set(syms) == {"mlxq_quantized_matmul", "mlxq_gather_qmm", "mlxq_dequantize", "mlxq_last_error"}

    def nargs(decl):
        inner = decl[decl.index("(") + 1:decl.rindex(")")]
        return 0 if inner.strip() in ("", "void") else inner.count(",") + 1

    fn_types = {"mlxq_quantized_matmul": "QmmFn", "mlxq_gather_qmm": "GatherFn", "mlxq_dequantize": "DequantFn"}
    for sym, ty in fn_types.items():
        m = re.search(r"^\+using " + ty + r" = int \(\*\)\((.*?)\);", text, re.M | re.S)
        assert m, ty
        patch_args = re.sub(r"\n\+\s*", " ", m.group(1)).count(",") + 1
        h = re.search(r"mlxq_status " + sym + r"\((.*?)\);", header, re.S)
        assert h, sym
        assert patch_args == h.group(1).count(",") + 1, sym
