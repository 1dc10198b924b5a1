"""The JAX drop-in (train-gpt_amd/jax_ops.py) against the XLA FFI handlers it
calls, checked on the CPU as source: jax is not installed in this image, so
the module is compiled, not imported.  Every jax.ffi call must name a
registered target, pass as many operands and request as many results as the
target's handler binds (.Arg / .Ret in csrc/ffi/tg_xla_ffi.cc), and pass
exactly the handler's attributes by name.  The custom_vjp wiring must match
the reference's (fp8.py:30-36,81-101; kernels.py:55,101-120)."""
import ast
import os
import py_compile
import re

import build
import xla_ffi

SRC = os.path.join(os.path.dirname(build.FFI_SRC), "..", "..", "jax_ops.py")


def _handler_bindings():
    """exported handler symbol -> (n_args, n_rets, attr names) from the FFI source."""
    text = open(build.FFI_SRC).read()
    out = {}
    for m in re.finditer(r"XLA_FFI_DEFINE_HANDLER_SYMBOL\(\s*(tg_ffi_\w+)\s*,\s*\w+\s*,(.*?)\);", text, re.S):
        body = m.group(2)
        out[m.group(1)] = (len(re.findall(r"\.Arg<", body)), len(re.findall(r"\.Ret<", body)),
                           sorted(re.findall(r'\.Attr<[^>]*>\("(\w+)"\)', body)))
    return out


def _calls(tree):
    """(target, n_operands, n_results, attr names) of every _call(...) in the module."""
    out = []
    for node in ast.walk(tree):
        if isinstance(node, ast.Call) and isinstance(node.func, ast.Name) and node.func.id == "_call":
            target = node.args[0].value
            shapes = node.args[1]
            n_res = len(shapes.elts) if isinstance(shapes, ast.Tuple) else 1
            out.append((target, len(node.args) - 2, n_res, sorted(k.arg for k in node.keywords)))
    return out


def test_module_compiles():
    py_compile.compile(SRC, doraise=True)


def test_every_call_matches_its_handler():
    tree = ast.parse(open(SRC).read())
    calls = _calls(tree)
    bindings = _handler_bindings()
    assert len(calls) >= 7
    for target, n_ops, n_res, attrs in calls:
        assert target in xla_ffi.HANDLERS, target
        sym = xla_ffi.HANDLERS[target][0]
        n_args, n_rets, want_attrs = bindings[sym]
        assert (n_ops, n_res, attrs) == (n_args, n_rets, want_attrs), (target, (n_ops, n_res, attrs),
                                                                       (n_args, n_rets, want_attrs))
    # the reference's compute paths all reach a handler
    used = {c[0] for c in calls}
    for t in ("tg_block_scaled_matmul", "tg_block_scaled_matmul_bwd_bf16", "tg_block_scaled_matmul_bwd_fp8",
              "tg_quantize_rows", "tg_rms_norm", "tg_rms_norm_bwd", "tg_rms_norm_fp8"):
        assert t in used, t


def test_custom_vjp_wiring_is_the_references():
    text = open(SRC).read()
    tree = ast.parse(text)
    funcs = {n.name: n for n in tree.body if isinstance(n, ast.FunctionDef)}
    # block_scaled_matmul(a, b, block_k=128) and rms_norm(x, scale, eps): custom_vjp, nondiff arg 2
    for name, args in (("block_scaled_matmul", ["a", "b", "block_k"]), ("rms_norm", ["x", "scale", "eps"])):
        f = funcs[name]
        assert [a.arg for a in f.args.args] == args, name
        deco = ast.unparse(f.decorator_list[0])
        assert "jax.custom_vjp" in deco and "nondiff_argnums=(2,)" in deco, (name, deco)
    assert "block_scaled_matmul.defvjp(_fp8_forward_with_residuals, _fp8_backward)" in text
    assert "rms_norm.defvjp(_rms_norm_fwd, _rms_norm_bwd)" in text
    # backward signatures: (nondiff, residuals, g), residuals = the forward's un-quantized operands
    assert [a.arg for a in funcs["_fp8_backward"].args.args] == ["block_k", "residuals", "g"]
    assert [a.arg for a in funcs["_rms_norm_bwd"].args.args] == ["eps", "residuals", "g"]
    assert "return _fp8_forward(a, b, block_k), (a, b)" in text
    assert "return _rms_norm_pure(x, scale, eps), (x, scale)" in text
    # the reference's ValueError texts (fp8.py:53-56)
    assert 'raise ValueError(f"contracted-dim mismatch: a K={K}, b K={K_b}")' in text
    assert 'raise ValueError(f"K={K} not divisible by block_k={block_k}")' in text
