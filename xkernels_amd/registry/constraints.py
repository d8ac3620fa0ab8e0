"""Decidable constraint predicates of Op Specs (e.g. ``"K % 32 == 0"``).

Same mini-language as the reference's registry/constraints.py: numbers, bound
symbol names, arithmetic, comparisons, ``and``/``or``/``not`` and the
``dtype(x)`` builtin. Anything else is rejected at ingest as undecidable; an
unbound symbol at query time raises ``UndecidableConstraintError`` so callers
can skip (not reject) the constraint.
"""
from __future__ import annotations

import ast
import operator
from typing import Any


class UndecidableConstraintError(ValueError):
    """The constraint uses syntax outside the decidable subset, or an unbound name."""


_BIN = {ast.Add: operator.add, ast.Sub: operator.sub, ast.Mult: operator.mul,
        ast.Mod: operator.mod, ast.FloorDiv: operator.floordiv, ast.Div: operator.truediv}
_CMP = {ast.Eq: operator.eq, ast.NotEq: operator.ne, ast.Lt: operator.lt,
        ast.LtE: operator.le, ast.Gt: operator.gt, ast.GtE: operator.ge}


def _parse(expr: str) -> ast.Expression:
    try:
        tree = ast.parse(expr, mode="eval")
    except SyntaxError as e:
        raise UndecidableConstraintError(f"unparseable constraint {expr!r}: {e}") from e
    for node in ast.walk(tree):
        ok = isinstance(node, (ast.Expression, ast.BoolOp, ast.UnaryOp, ast.BinOp, ast.Compare,
                               ast.Constant, ast.Name, ast.Call, ast.Load, ast.And, ast.Or,
                               ast.Not, ast.USub, *_BIN, *_CMP))
        if not ok:
            raise UndecidableConstraintError(f"{expr!r}: {type(node).__name__} not allowed")
        if isinstance(node, ast.Call):
            if not (isinstance(node.func, ast.Name) and node.func.id == "dtype"
                    and len(node.args) == 1 and isinstance(node.args[0], ast.Name)):
                raise UndecidableConstraintError(f"{expr!r}: only dtype(<name>) calls are allowed")
    return tree


def validate_decidable(expr: str) -> None:
    _parse(expr)


def _eval(node, b: dict[str, Any]):
    if isinstance(node, ast.Expression):
        return _eval(node.body, b)
    if isinstance(node, ast.Constant):
        return node.value
    if isinstance(node, ast.Name):
        if node.id not in b:
            raise UndecidableConstraintError(f"unbound symbol {node.id!r}")
        return b[node.id]
    if isinstance(node, ast.Call):
        key = f"dtype:{node.args[0].id}"
        if key not in b:
            raise UndecidableConstraintError(f"unbound dtype of {node.args[0].id!r}")
        return b[key]
    if isinstance(node, ast.UnaryOp):
        v = _eval(node.operand, b)
        return (not v) if isinstance(node.op, ast.Not) else -v
    if isinstance(node, ast.BinOp):
        return _BIN[type(node.op)](_eval(node.left, b), _eval(node.right, b))
    if isinstance(node, ast.BoolOp):
        vals = [_eval(v, b) for v in node.values]
        return all(vals) if isinstance(node.op, ast.And) else any(vals)
    if isinstance(node, ast.Compare):
        left = _eval(node.left, b)
        for op, comp in zip(node.ops, node.comparators):
            right = _eval(comp, b)
            if not _CMP[type(op)](left, right):
                return False
            left = right
        return True
    raise UndecidableConstraintError(f"cannot evaluate {type(node).__name__}")


def evaluate(expr: str, bindings: dict[str, Any]) -> bool:
    return bool(_eval(_parse(expr), bindings))
