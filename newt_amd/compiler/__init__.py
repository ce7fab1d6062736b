"""The newt compiler for gfx950: kernel AST -> HIP C++ source."""

from .codegen import CompileError, Codegen, _Retry
from .ops_dot import DotOps
from .ops_memory import MemoryOps
from .ops_pipeline import DotPipeline
from .ops_reduce import ReduceOps


class Param:
    """A runtime kernel parameter as specialized by the JIT: its dtype (or
    pointer type), C name, and the value facts compiled into the kernel
    (integer == 1, power-of-two divisor up to 16, pointer 16-byte aligned)."""

    def __init__(self, dtype, cname, eq1=False, div=1, aligned16=False):
        self.dtype = dtype
        self.cname = cname
        self.eq1 = eq1
        self.div = div
        self.aligned16 = aligned16

    def __repr__(self):
        return f"Param({self.dtype}, {self.cname}, eq1={self.eq1}, div={self.div}, a16={self.aligned16})"


class Compiler(DotPipeline, DotOps, ReduceOps, MemoryOps, Codegen):
    pass


def _has_row_reduction(fndef):
    import ast
    for n in ast.walk(fndef):
        if isinstance(n, ast.Call):
            name = n.func.attr if isinstance(n.func, ast.Attribute) else getattr(n.func, "id", None)
            if name in ("sum", "max", "min"):
                for kw in n.keywords:
                    if kw.arg == "axis" and isinstance(kw.value, ast.Constant) and kw.value.value in (1, -1):
                        return True
                if len(n.args) >= 2 and isinstance(n.args[1], ast.Constant) and n.args[1].value in (1, -1):
                    return True
    return False


def compile_fn(fndef, fn_globals, params, constexprs, num_warps, kernel_name, num_stages=3,
               max_passes=10):
    """Compile a kernel. Returns (hip_source, lds_bytes).

    params: list of (name, Param) for the runtime parameters in signature order.
    Mirrors the reference boundary compile_fn(...) -> (source, smem)
    (newt/compiler/codegen.py:2758-2765); layout hints learned by one pass are
    fed to the next until no new hint appears."""
    hints = {}
    prefer_rows = _has_row_reduction(fndef)
    last = None
    for _ in range(max_passes):
        cg = Compiler(fndef, fn_globals, params, constexprs, num_warps, kernel_name,
                      num_stages=num_stages, hints=hints)
        cg.prefer_rows = prefer_rows
        try:
            src = cg.compile()
        except _Retry:
            hints.update(cg.new_hints)
            continue
        fresh = {k: v for k, v in cg.new_hints.items() if hints.get(k) != v}
        last = (src, cg.lds_total)
        if not fresh:
            return last
        hints.update(fresh)
    if last is None:
        raise CompileError(f"{fndef.name}: layout assignment did not converge")
    return last


__all__ = ["CompileError", "Param", "compile_fn", "Compiler"]
