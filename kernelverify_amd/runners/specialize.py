"""Fill a kernel template's `$NAME` holes and return a concrete `KernelSpec`.

The runner door's template mechanism (the reference's
kernelverify/runners/specialize.py:29-70 is the interface: same function
name, arguments and failure type). A template is an ordinary `KernelSpec`
whose `source`, `entry_point` or `name` text contains placeholders, written
`$NAME` or `${NAME}`; `$$` stands for a literal dollar sign. HIP C++ source
and the pack-library descriptors use `$` only this way.

One scan finds every placeholder of the three texts; then two kinds of
mistake are reported together, each as a `SpecError` that lists every name
involved:

- holes the substitutions leave empty;
- substitutions no hole asks for (a misspelled key looks exactly like this).

Values are rendered with `str()`. Bindings and launch shape are carried over
unchanged, and the result is validated by `KernelSpec` itself.
"""

from __future__ import annotations

import re

from kernelverify_amd.runners.spec import KernelSpec, SpecError

# `$$` (escape), `$NAME`, `${NAME}`, or a `$` followed by anything else (an error)
_HOLE = re.compile(r"\$(?:(\$)|([A-Za-z_]\w*)|\{([A-Za-z_]\w*)\}|(.?))", re.S)

_TEXT_FIELDS = ("source", "entry_point", "name")


def placeholders(text: str) -> list[str]:
    """The placeholder names of ``text`` in order of first appearance."""
    seen: dict[str, None] = {}
    for m in _HOLE.finditer(text):
        name = m.group(2) or m.group(3)
        if name:
            seen.setdefault(name, None)
    return list(seen)


def _fill(text: str, values: dict, where: str) -> str:
    def one(m: re.Match) -> str:
        if m.group(1):
            return "$"
        name = m.group(2) or m.group(3)
        if name is None:
            raise SpecError(f"{where}: a '$' at offset {m.start()} opens no placeholder "
                            "(write $$ for a literal dollar sign)")
        return str(values[name])

    return _HOLE.sub(one, text)


def specialize(template: KernelSpec, substitutions: dict) -> KernelSpec:
    """A validated `KernelSpec` with every placeholder of ``template`` filled
    from ``substitutions``."""
    texts = {f: getattr(template, f) for f in _TEXT_FIELDS}
    wanted = {f: placeholders(t) for f, t in texts.items()}
    asked = {n for names in wanted.values() for n in names}
    empty = sorted(asked - set(substitutions))
    stray = sorted(set(substitutions) - asked)
    problems = []
    if empty:
        where = {n: [f for f in _TEXT_FIELDS if n in wanted[f]] for n in empty}
        problems.append("no value for " + ", ".join(
            f"${n} (in {'/'.join(where[n])})" for n in empty))
    if stray:
        problems.append(f"values for {stray} fill no placeholder (is a key misspelled?)")
    if problems:
        raise SpecError(f"specialize {template.name or template.entry_point!r}: "
                        + "; ".join(problems))
    filled = {f: _fill(t, substitutions, f) for f, t in texts.items()}
    return KernelSpec(source=filled["source"], entry_point=filled["entry_point"],
                      bindings=template.bindings, launch=template.launch, name=filled["name"])
