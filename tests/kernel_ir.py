"""A reader of the reference's printed Kernel IR (crates/modelspec-core/src/ir/kernel.rs:1407-1560,
print format of crates/modelspec-cli/tests/golden/*.kernel.ir): buffers, bindings, kernels (fusion
groups) and the step and forward plans, and of this backend's plan text (msx_plan)."""
import re


def parse_reference(text):
    """{'buffers': {name: bytes}, 'kernels': {id: {'kind', 'ops', 'epilogue', 'transposed'}},
    'plans': {'step' | 'forward': [{'kernel', 'value', 'reads', 'writes'}]}, 'bindings': [...]}"""
    out = {"buffers": {}, "kernels": {}, "plans": {}, "bindings": []}
    plan = None
    for line in text.splitlines():
        m = re.match(r"buffer (b\d+): (\d+) bytes$", line)
        if m:
            out["buffers"][m.group(1)] = int(m.group(2))
            continue
        m = re.match(r"(input|target|param|loss|prediction) (.*)$", line)
        if m and plan is None:
            out["bindings"].append((m.group(1), m.group(2)))
            continue
        m = re.match(r"kernel (k\d+) \S+ (\w+) (\S+) f32 \((.*)\) -> (Tensor<[^>]*>)(.*)$", line)
        if m:
            kid, kind, ops, args, result, rest = m.groups()
            epi = re.search(r"epilogue (\w+)", rest)
            out["kernels"][kid] = {"kind": kind, "ops": ops.split(">"), "epilogue": epi.group(1) if epi else None,
                                   "transposed": "transposed" in args, "result": result}
            continue
        m = re.match(r"plan (\w+)$", line)
        if m:
            plan = m.group(1)
            out["plans"][plan] = []
            continue
        m = re.match(r"\s+\d+: dispatch (k\d+) %(\d+) reads (.*?) writes (.*?) workgroups", line)
        if m and plan:
            kid, value, reads, writes = m.groups()
            buf = lambda s: re.findall(r"(b\d+)\[", s)
            out["plans"][plan].append({"kernel": kid, "value": int(value), "reads": buf(reads), "writes": buf(writes)})
    return out


def parse_plan(text):
    """This backend's plans: {'step' | 'forward': {'launches': [{'what', 'values', 'side'}],
    'arena': bytes, 'slices': {value: offset}}}."""
    out, plan = {}, None
    for line in text.splitlines():
        m = re.match(r"plan (\w+) \(\d+ launches\)$", line)
        if m:
            plan = m.group(1)
            out[plan] = {"launches": [], "arena": 0, "slices": {}}
            continue
        m = re.match(r"\s+\d+: (.*?)( \[side\])? flop \S+ bytes \S+$", line)
        if m:
            what = m.group(1)
            out[plan]["launches"].append({"what": what, "side": bool(m.group(2)),
                                          "values": [int(v) for v in re.findall(r"%(\d+)", what)]})
            continue
        m = re.match(r"\s+arena (\d+) bytes, \d+ values(.*)$", line)
        if m:
            out[plan]["arena"] = int(m.group(1))
            out[plan]["slices"] = {int(v): int(o) for v, o in re.findall(r"%(\d+)@(\d+)", m.group(2))}
    return out
