"""The integration guide at the repository root (the reference-side bindings a
maintainer adds) names only symbols this repository has in its code snippets: every
``aster_amd`` import resolves, every name the reference-side stub module re-exports
(``aster.optimization.hip_int8_paged``) is one of that stub's imports, the calls the
snippets make pass keyword arguments the functions accept, and every C entry point
the text mentions is declared in include/aster_kv.h."""

import ast
import importlib
import inspect
import os
import re

from tests.test_capi import declared_symbols

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOC = os.path.join(ROOT, "INTEGRATION.md")
STUB = "aster.optimization.hip_int8_paged"  # the module the doc asks the maintainer to add


def _blocks():
    text = open(DOC).read()
    return text, re.findall(r"```python\n(.*?)```", text, flags=re.S)


def _parse(code):
    """A snippet as a module (snippets that are method-body excerpts are dedented and
    wrapped so that ``return`` parses)."""
    body = "\n".join("    " + line for line in code.splitlines())
    return ast.parse("def _snippet(self):\n" + body + "\n")


def _resolve(module, name):
    return getattr(importlib.import_module(module), name)


def test_every_snippet_parses():
    _, blocks = _blocks()
    assert len(blocks) >= 5
    for code in blocks:
        _parse(code)


def test_imports_resolve_and_stub_names_are_its_imports():
    _, blocks = _blocks()
    stub = {}  # name the stub exports -> (aster_amd module, attribute)
    for code in blocks:
        for node in ast.walk(_parse(code)):
            if isinstance(node, ast.ImportFrom) and (node.module or "").startswith("aster_amd"):
                for alias in node.names:
                    target = _resolve(node.module, alias.name)
                    assert target is not None
                    stub[alias.asname or alias.name] = target
    assert {"bind_hip_backend", "hip_forward", "hip_forward_features",
            "HipPagedStateArchive"} <= set(stub)
    for code in blocks:
        for node in ast.walk(_parse(code)):
            if isinstance(node, ast.ImportFrom) and node.module == STUB:
                for alias in node.names:
                    assert alias.name in stub, alias.name


def _callee(node, names):
    if isinstance(node.func, ast.Name):
        return names.get(node.func.id)
    return None


def test_calls_use_accepted_keywords():
    from aster_amd import PagedKVCache
    from aster_amd.runner import PagedAttentionStep

    _, blocks = _blocks()
    names = {}
    for code in blocks:
        for node in ast.walk(_parse(code)):
            if isinstance(node, ast.ImportFrom) and (node.module or "").startswith("aster_amd"):
                for alias in node.names:
                    names[alias.asname or alias.name] = _resolve(node.module, alias.name)
    names.update({
        "bind_hip_backend": _resolve("aster_amd.runner", "bind_hip_backend"),
        "hip_forward": _resolve("aster_amd.runner", "hip_forward"),
        "hip_forward_features": _resolve("aster_amd.runner", "hip_forward_features"),
        "HipPagedStateArchive": _resolve("aster_amd.offload", "PagedStateArchive"),
    })
    methods = {"attend": PagedAttentionStep.attend, "paged_attention": PagedKVCache.paged_attention}
    checked = 0
    for code in blocks:
        for node in ast.walk(_parse(code)):
            if not isinstance(node, ast.Call):
                continue
            fn = _callee(node, names)
            if fn is None and isinstance(node.func, ast.Attribute):
                fn = methods.get(node.func.attr)
            if fn is None:
                continue
            params = inspect.signature(fn).parameters
            if any(p.kind is p.VAR_KEYWORD for p in params.values()):
                params = {**params, **inspect.signature(
                    _resolve("aster_amd.runner", "bind_hip_backend")).parameters}
            for kw in node.keywords:
                if kw.arg is not None:
                    assert kw.arg in params, (getattr(fn, "__qualname__", fn), kw.arg)
            checked += 1
    assert checked >= 8


def test_reference_binding_keeps_the_reference_class():
    """The binding the doc shows, run on a stand-in for the reference's class: the
    instance keeps its own class (the gate of adapters.py:47-50 compares types) and
    gets the attributes the reference's constructor sets."""
    import torch

    from aster_amd.runner import bind_hip_backend
    from tests.llama_like import LlamaLike

    class PagedAttentionRunner:  # stand-in: only its identity matters here
        pass

    runner = bind_hip_backend(PagedAttentionRunner(), LlamaLike(seed=0),
                              policy_artifact_id="p", backend="hip_int8_paged")
    assert type(runner) is PagedAttentionRunner
    for name in ("model", "pool", "codec", "policy_artifact_id", "tokenizer", "chat_template",
                 "device", "query_block_size", "key_block_size", "attention_fallback",
                 "attention_work", "backend", "input_tokens_computed", "forward_calls",
                 "model_execution_seconds"):
        assert hasattr(runner, name), name
    assert runner.backend == "hip_int8_paged" and runner.device == torch.device("cpu")


def test_mentioned_entry_points_are_declared():
    text, _ = _blocks()
    declared = set(declared_symbols())
    with open(os.path.join(ROOT, "include", "aster_kv.h")) as f:
        structs = set(re.findall(r"typedef struct (astr_\w+)", f.read()))
    for name in set(re.findall(r"\bastr_\w+", text)):
        if name in structs:  # the arena descriptor, the plan's record
            continue
        stem = name.rstrip("_")
        assert stem in declared or any(d.startswith(stem) for d in declared), name
