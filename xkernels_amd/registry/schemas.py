"""JSON-Schema documents for Op Specs / Impl Cards and a validator.

``jsonschema`` is used when importable; otherwise a built-in validator covering
the keywords the two schemas use (type, required, properties,
additionalProperties, enum, pattern, items, minimum, minProperties, $ref to
$defs) runs instead, so structural checks never silently disappear.
"""
from __future__ import annotations

import json
import re
from functools import cache
from pathlib import Path

_REGISTRY_ROOT = Path(__file__).resolve().parents[2] / "registry"

try:  # pragma: no cover - optional dependency
    import jsonschema  # type: ignore[import-untyped]

    _HAVE_JSONSCHEMA = True
except Exception:  # noqa: BLE001
    _HAVE_JSONSCHEMA = False


def registry_root() -> Path:
    return _REGISTRY_ROOT


@cache
def _schema(name: str) -> dict:
    with (_REGISTRY_ROOT / "schema" / name).open() as f:
        return json.load(f)


def op_spec_schema() -> dict:
    return _schema("op_spec.schema.json")


def impl_card_schema() -> dict:
    return _schema("impl_card.schema.json")


def have_validator() -> bool:
    return _HAVE_JSONSCHEMA


class SchemaError(ValueError):
    pass


_TYPES = {
    "object": dict, "array": list, "string": str, "boolean": bool,
    "integer": int, "number": (int, float), "null": type(None),
}


def _type_ok(value, t) -> bool:
    if isinstance(t, list):
        return any(_type_ok(value, x) for x in t)
    if t in ("integer", "number") and isinstance(value, bool):
        return False
    return isinstance(value, _TYPES[t])


def _check(inst, sch: dict, root: dict, path: str) -> None:
    if "$ref" in sch:
        ref = sch["$ref"]
        if not ref.startswith("#/"):
            raise SchemaError(f"{path}: unsupported $ref {ref}")
        node = root
        for part in ref[2:].split("/"):
            node = node[part]
        _check(inst, node, root, path)
        return
    if "type" in sch and not _type_ok(inst, sch["type"]):
        raise SchemaError(f"{path}: expected {sch['type']}, got {type(inst).__name__}")
    if "enum" in sch and inst not in sch["enum"]:
        raise SchemaError(f"{path}: {inst!r} not in {sch['enum']}")
    if "pattern" in sch and isinstance(inst, str) and not re.search(sch["pattern"], inst):
        raise SchemaError(f"{path}: {inst!r} does not match {sch['pattern']}")
    if "minimum" in sch and isinstance(inst, (int, float)) and inst < sch["minimum"]:
        raise SchemaError(f"{path}: {inst} < {sch['minimum']}")
    if isinstance(inst, dict):
        for r in sch.get("required", []):
            if r not in inst:
                raise SchemaError(f"{path}: missing required {r!r}")
        if "minProperties" in sch and len(inst) < sch["minProperties"]:
            raise SchemaError(f"{path}: fewer than {sch['minProperties']} properties")
        props = sch.get("properties", {})
        addl = sch.get("additionalProperties", True)
        for k, v in inst.items():
            if k in props:
                _check(v, props[k], root, f"{path}.{k}")
            elif addl is False:
                raise SchemaError(f"{path}: unexpected property {k!r}")
            elif isinstance(addl, dict):
                _check(v, addl, root, f"{path}.{k}")
    if isinstance(inst, list) and isinstance(sch.get("items"), dict):
        for i, v in enumerate(inst):
            _check(v, sch["items"], root, f"{path}[{i}]")


def validate(doc: dict, schema: dict) -> None:
    if _HAVE_JSONSCHEMA:  # pragma: no cover
        jsonschema.validate(instance=doc, schema=schema)
    else:
        _check(doc, schema, schema, "$")


def validate_op_spec(doc: dict) -> None:
    validate(doc, op_spec_schema())


def validate_impl_card(doc: dict) -> None:
    validate(doc, impl_card_schema())
