"""Turn a kernel template into a concrete `KernelSpec` (reference:
kernelverify/runners/specialize.py:29-70).

A template is an ordinary `KernelSpec` whose source, entry point or name hold
`$NAME` placeholders. `specialize` fills them from a dict and returns a new,
validated spec; bindings and launch pass through. A placeholder left unfilled
raises, and so does a substitution the template never mentions (almost
always a misspelled name). `$` appears in neither HIP C++ kernels nor the
pack-library descriptors except as a placeholder.
"""

from __future__ import annotations

from string import Template

from kernelverify_amd.runners.spec import KernelSpec, SpecError


def _identifiers(parsed: Template) -> set:
    """The `$NAME` / `${NAME}` placeholders of a template (what
    Template.get_identifiers gives on Python 3.11+)."""
    names = set()
    for match in parsed.pattern.finditer(parsed.template):
        name = match.group("named") or match.group("braced")
        if name:
            names.add(name)
    return names


def specialize(template: KernelSpec, substitutions: dict) -> KernelSpec:
    texts = {"source": template.source, "entry_point": template.entry_point,
             "name": template.name}
    used: set = set()
    filled: dict = {}
    for where, text in texts.items():
        parsed = Template(text)
        used.update(_identifiers(parsed))
        try:
            filled[where] = parsed.substitute(substitutions)
        except KeyError as error:
            raise SpecError(f"the template's {where} names ${error.args[0]}, "
                            "which the substitutions do not supply") from error
        except ValueError as error:
            raise SpecError(f"the template's {where} is malformed: {error}") from error
    unused = sorted(set(substitutions) - used)
    if unused:
        raise SpecError(f"substitutions {unused} appear nowhere in the template; "
                        "a misspelled placeholder name looks exactly like this")
    return KernelSpec(source=filled["source"], entry_point=filled["entry_point"],
                      bindings=template.bindings, launch=template.launch, name=filled["name"])
