"""The calls INTEGRATION.md shows a maintainer agree with the prototypes of include/qmm.h: every `qmm_*(...)` call
in the document names a declared entry point, passes as many arguments as it declares (a `...` stands for a run of
arguments: those before it line up from the front, those after it from the back), and every argument spelled as one
of the prototype's parameter names sits at that parameter's position (or is passed there as well). A call written
in an older argument order fails here."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qmm.h")
DOC = os.path.join(ROOT, "INTEGRATION.md")


def prototypes():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"^(?:int|int64_t|const char \*)\s*(qmm_\w+)\(([^)]*)\);", text, flags=re.M):
        params = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        out[m.group(1)] = [re.findall(r"\w+", p)[-1] for p in params]
    return out


def split_args(body):
    """Top-level comma split of a call's argument text."""
    args, depth, cur = [], 0, ""
    for ch in body:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            args.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        args.append(cur.strip())
    return args


def doc_calls():
    """(line number, function name, argument list) of every qmm_*(...) call with arguments in the document."""
    text = open(DOC).read()
    out = []
    for m in re.finditer(r"\b(qmm_\w+)\(", text):
        i, depth = m.end(), 1
        while i < len(text) and depth:
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        body = text[m.end():i - 1]
        if body.strip():
            out.append((text.count("\n", 0, m.start()) + 1, m.group(1), split_args(body)))
    return out


def test_document_has_calls():
    assert len(doc_calls()) >= 30


def test_every_call_matches_its_prototype():
    protos = prototypes()
    bad = []
    for line, name, args in doc_calls():
        if name not in protos:
            bad.append(f"INTEGRATION.md:{line}: {name} is not declared in include/qmm.h")
            continue
        params = protos[name]
        if "..." in args:
            cut = args.index("...")
            head, tail = args[:cut], args[cut + 1:]
            if len(head) + len(tail) > len(params):
                bad.append(f"INTEGRATION.md:{line}: {name} has {len(head) + len(tail)} arguments around '...', "
                           f"the prototype {len(params)}")
                continue
            placed = list(enumerate(head)) + [(len(params) - len(tail) + j, a) for j, a in enumerate(tail)]
        else:
            if len(args) != len(params):
                bad.append(f"INTEGRATION.md:{line}: {name} has {len(args)} arguments, the prototype {len(params)}")
                continue
            placed = list(enumerate(args))
        at = dict(placed)
        for pos, a in placed:
            # a value passed for two parameters (the down GEMM's max_rows as x_rows) is fine where it also sits at its own
            if re.fullmatch(r"[A-Za-z_]\w*", a) and a in params and params.index(a) != pos and \
                    at.get(params.index(a)) != a:
                bad.append(f"INTEGRATION.md:{line}: {name} passes '{a}' at position {pos}, the prototype declares "
                           f"it at {params.index(a)}")
    assert not bad, "\n".join(bad)


def test_checker_catches_a_shifted_call():
    """The old qmm_moe_grouped order (max_tiles before E, KU) is caught."""
    params = prototypes()["qmm_moe_grouped"]
    old = split_args("QMM_Q4_K, 0, fused, act, max_tiles, H, FE, E, KU, tile_info, rowmap, x16, QMM_F16, s_h, t, wg, "
                     "NULL, wu, NULL, NULL, NULL, act_sorted, stream")
    assert len(old) == len(params)
    assert any(a in params and params.index(a) != i for i, a in enumerate(old))


def test_every_entry_point_is_documented():
    """Every entry point the header declares has at least one call in the document."""
    doc = open(DOC).read()
    missing = [name for name in prototypes() if not re.search(rf"\b{name}\(", doc)]
    assert not missing, f"entry points without a call in INTEGRATION.md: {missing}"
