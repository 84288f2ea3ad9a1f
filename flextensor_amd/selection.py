"""Which modules become offload units: include and exclude patterns.

The rules are the reference's (tensor_discovery.py:470-569; utils.py:148-406;
offload_manager.py:2725-2806):

* A pattern is split on dots and each segment is a shell-style glob over one
  path segment (``*`` any run of characters, ``?`` one character).
* A segment that is exactly ``*`` matches one segment when module paths are
  selected by an include pattern, and one or more segments when module
  paths are excluded or parameter paths are matched.
* ``class:<glob>`` matches a module's class by its short name or its fully
  qualified name (``module.qualname``), with ``*`` spanning dots there.
  ``name:<glob>`` is a plain path pattern. Empty bodies are refused.
* An include pattern may name parameters (``layers.*.weight``). It is
  truncated from the right to the longest prefix that matches a module path;
  if no prefix does, the modules owning the matched parameters are used.
  A prefix that matches a module while the full pattern names no parameter
  selects nothing, so an unmatched name cannot widen to an ancestor.
* The outermost matching modules are the units, in module order. A matched
  ``ModuleList`` / ``ModuleDict`` stands for its children, whose forwards
  are the ones that run; this departs from the reference, which would patch
  the container itself.
* Excludes then drop units. Patterns that match nothing log a warning; an
  include list that yields no unit logs an error.
"""

from __future__ import annotations

import functools
import logging
import re
from collections.abc import Callable, Sequence

from torch import nn

LOGGER = logging.getLogger(__name__)

CLASS_PREFIX = "class:"
NAME_PREFIX = "name:"


@functools.lru_cache(maxsize=4096)
def _glob(segment: str) -> re.Pattern[str]:
    return re.compile("".join(".*" if c == "*" else "." if c == "?" else re.escape(c) for c in segment))


def _match(parts: tuple[str, ...], pats: tuple[str, ...], recursive: bool) -> bool:
    if not pats:
        return not parts
    if not parts:
        return False
    head = pats[0]
    if head == "*" and recursive:
        return any(_match(parts[i + 1:], pats[1:], recursive) for i in range(len(parts)))
    return _glob(head).fullmatch(parts[0]) is not None and _match(parts[1:], pats[1:], recursive)


def path_matches(path: str, pattern: str, *, recursive_star: bool) -> bool:
    """Whether the dotted ``path`` matches ``pattern`` (``recursive_star``: a lone ``*`` spans segments)."""
    return _match(tuple(path.split(".")), tuple(pattern.split(".")), recursive_star)


def partition(patterns: Sequence[str]) -> tuple[list[str], list[str]]:
    """``(path patterns, class patterns)`` with the ``name:`` / ``class:`` prefixes removed."""
    names: list[str] = []
    classes: list[str] = []
    for p in patterns:
        for prefix, into in ((CLASS_PREFIX, classes), (NAME_PREFIX, names)):
            if p.startswith(prefix):
                body = p[len(prefix):]
                if not body.strip():
                    raise ValueError(f"pattern {p!r} has an empty body; use {prefix}<glob> or remove the entry")
                into.append(body)
                break
        else:
            names.append(p)
    return names, classes


def class_matches(cls: type, patterns: Sequence[str]) -> bool:
    short, full = cls.__name__, f"{cls.__module__}.{cls.__qualname__}"
    return any(_glob(p).fullmatch(short) or _glob(p).fullmatch(full) for p in patterns)


def _param_paths(model: nn.Module, pattern: str) -> list[str]:
    return [n for n, _ in model.named_parameters() if path_matches(n, pattern, recursive_star=True)]


def module_patterns(patterns: Sequence[str], module_paths: Sequence[str], model: nn.Module | None) -> list[str]:
    """Module-level patterns for include patterns that may name parameters (tensor_discovery.py:484-535)."""
    known = set(module_paths)
    out: dict[str, None] = {}
    for pattern in patterns:
        parts = pattern.split(".")
        prefix_matched = False
        for n in range(len(parts), 0, -1):
            cand = ".".join(parts[:n])
            if n < len(parts) and cand == "*":
                continue
            if not any(path_matches(m, cand, recursive_star=False) for m in module_paths):
                continue
            prefix_matched = True
            if n == len(parts) or model is None or _param_paths(model, pattern):
                out[cand] = None
            break
        if not prefix_matched and model is not None:
            for p in _param_paths(model, pattern):
                parent = p.rpartition(".")[0]
                if parent in known:
                    out[parent] = None
    return list(out)


def _pattern_matched(model: nn.Module, pattern: str, module_paths: Sequence[str], recursive: bool) -> bool:
    names, classes = partition([pattern])
    if classes:
        return any(class_matches(type(m), classes) for p, m in model.named_modules() if p)
    return (any(path_matches(m, names[0], recursive_star=recursive) for m in module_paths)
            or bool(_param_paths(model, names[0])))


def prefix_matches(path: str, patterns: Sequence[str]) -> bool:
    """Whether a prefix of the dotted ``path`` (the whole path included) matches one of the path
    ``patterns``, a lone ``*`` spanning segments (tensor_discovery.py:288-307): a module pattern
    covers every parameter below that module."""
    parts = path.split(".")
    return any(path_matches(".".join(parts[:i]), p, recursive_star=True)
               for i in range(1, len(parts) + 1) for p in patterns)


def parameter_filter(model: nn.Module, include: Sequence[str], exclude: Sequence[str]) -> Callable[[str], bool]:
    """``path -> bool``: whether the parameter at ``path`` is streamed with its unit.

    Included when a prefix of its path matches an include path pattern or an
    ancestor module's class matches an include ``class:`` pattern; dropped
    when an exclude pattern matches the same way (tensor_discovery.py:326-372,
    647-700). Parameters a unit does not stream stay on the GPU.
    """
    inc_names, inc_classes = partition(list(include) or ["*"])
    ex_names, ex_classes = partition(list(exclude))
    inc_paths = {p for p, m in model.named_modules() if p and inc_classes and class_matches(type(m), inc_classes)}
    ex_paths = {p for p, m in model.named_modules() if p and ex_classes and class_matches(type(m), ex_classes)}

    def under(path: str, paths: set[str]) -> bool:
        parts = path.split(".")
        return bool(paths) and any(".".join(parts[:i]) in paths for i in range(1, len(parts) + 1))

    def streamed(path: str) -> bool:
        if not (prefix_matches(path, inc_names) or under(path, inc_paths)):
            return False
        return not ((ex_names and prefix_matches(path, ex_names)) or under(path, ex_paths))

    return streamed


def select_offload_units(model: nn.Module, include: Sequence[str], exclude: Sequence[str]) -> list[str]:
    """Paths of the offload units of ``model`` for these patterns, in module order."""
    if not include:
        LOGGER.warning("include_patterns is an empty list; no module is patched. Use offload_block() for manual "
                       "offload units, or include_patterns=['*'] to include all.")
        return []
    module_paths = [p for p, _ in model.named_modules() if p]
    names, classes = partition(include)
    mods = module_patterns(names, module_paths, model)
    chosen: list[str] = []
    taken: set[str] = set()
    for path, mod in model.named_modules():
        if not path or path in taken or any(path.startswith(c + ".") for c in chosen):
            continue
        if not ((classes and class_matches(type(mod), classes))
                or any(path_matches(path, p, recursive_star=False) for p in mods)):
            continue
        if isinstance(mod, (nn.ModuleList, nn.ModuleDict)):
            children = [f"{path}.{c}" for c, _ in mod.named_children()]
            chosen.extend(children)
            taken.update(children)
            continue
        chosen.append(path)
        taken.add(path)
    for pattern in include:
        if not _pattern_matched(model, pattern, module_paths, recursive=False):
            LOGGER.warning("Include pattern '%s' did not match any modules or parameters.", pattern)
    ex_names, ex_classes = partition(exclude)
    kept = [p for p in chosen
            if not any(path_matches(p, x, recursive_star=True) for x in ex_names)
            and not (ex_classes and class_matches(type(model.get_submodule(p)), ex_classes))]
    for pattern in exclude:
        if not _pattern_matched(model, pattern, module_paths, recursive=True):
            LOGGER.warning("Exclude pattern '%s' did not match any modules or parameters.", pattern)
    if chosen and not kept:
        LOGGER.error("All %d included modules were removed by exclude_patterns %s. Offloading is effectively "
                     "disabled.", len(chosen), list(exclude))
    elif not chosen:
        LOGGER.error("No modules matched any include pattern %s. Offloading is effectively disabled. Check pattern "
                     "spelling against model.named_modules() paths.", list(include))
    return kept
