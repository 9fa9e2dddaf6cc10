"""pkg/ggufembed's Runtime over the GPU library: task prompts (tasks.go),
dimension resolution, tokenization and ONE batched forward for all inputs
(in place of embedPrompts' one-forward-per-prompt fan-out, api.go:237-295).

    rt = embed.open("embeddinggemma-300m-Q8_0.gguf")
    vecs = rt.embed(["hello world", ...])            # TaskSearchQuery, dim 512
    vec = rt.embed_single_input(EmbedInput(Task.SEARCH_DOCUMENT, "text", title="t", dim=768))
"""
from __future__ import annotations

import dataclasses
import enum
import os

import numpy as np

from . import _lib
from .runtime import Context, Model, resolve_dim  # noqa: F401  (resolve_dim is part of this API)
from .tokenizer import Tokenizer

# unicode.IsSpace (what strings.TrimSpace trims); Python's str.strip() would also
# trim U+001C..U+001F, which Go keeps.
_GO_SPACE = ("\t\n\v\f\r \x85\xa0\u1680\u2000\u2001\u2002\u2003\u2004\u2005\u2006\u2007\u2008\u2009"
             "\u200a\u2028\u2029\u202f\u205f\u3000")


class Task(enum.IntEnum):
    """ggufembed.Task (tasks.go:9-37)."""
    NONE = -1
    SEARCH_QUERY = 0
    SEARCH_DOCUMENT = 1
    QUESTION_ANSWERING = 2
    FACT_VERIFICATION = 3
    CLASSIFICATION = 4
    CLUSTERING = 5
    SEMANTIC_SIMILARITY = 6
    CODE_RETRIEVAL = 7


_DEFAULT_DESCRIPTIONS = {  # defaultTaskDescriptions, tasks.go:149-157
    Task.SEARCH_QUERY: "search result",
    Task.QUESTION_ANSWERING: "question answering",
    Task.FACT_VERIFICATION: "fact checking",
    Task.CLASSIFICATION: "classification",
    Task.CLUSTERING: "clustering",
    Task.SEMANTIC_SIMILARITY: "sentence similarity",
    Task.CODE_RETRIEVAL: "code retrieval",
}


class EmbedError(ValueError):
    pass


class Cancelled(EmbedError):
    """ctx.Err() of a cancelled context (context.Canceled): raised instead of
    starting the next unit of work."""


def _check_ctx(ctx):
    """The `select { case <-ctx.Done(): ... }` of EmbedSingleInput
    (pkg/ggufembed/api.go:190-195) and embedPrompts (:268-273).  ctx: None
    (never cancelled), an object with is_set() (threading.Event), or a
    callable returning True once cancelled."""
    if ctx is None:
        return
    if ctx.is_set() if hasattr(ctx, "is_set") else ctx():
        raise Cancelled("context canceled")


@dataclasses.dataclass
class EmbedInput:
    """ggufembed.EmbedInput (tasks.go:62-82)."""
    task: int = Task.SEARCH_QUERY
    content: str = ""
    title: str = ""
    custom_task_description: str = ""
    dim: int = 0


def build_prompt(inp: EmbedInput) -> str:
    """BuildPrompt / EmbedInput.prompt (tasks.go:117-147, 159-163)."""
    content = inp.content.strip(_GO_SPACE)
    if content == "":
        raise EmbedError("content must not be empty")
    if inp.task == Task.NONE:
        return content
    if inp.task == Task.SEARCH_DOCUMENT:
        title = inp.title.strip(_GO_SPACE) or "none"
        return f"title: {title} | text: {content}"
    desc = inp.custom_task_description.strip(_GO_SPACE)
    if desc == "":
        try:
            desc = _DEFAULT_DESCRIPTIONS[Task(inp.task)]
        except (KeyError, ValueError):
            raise EmbedError(f"unsupported task {_task_name(inp.task)} (missing default description)") from None
    return f"task: {desc} | query: {content}"


def _task_name(t) -> str:
    """Task.String (tasks.go:39-60)."""
    names = {-1: "none", 0: "search_query", 1: "search_document", 2: "question_answering",
             3: "fact_verification", 4: "classification", 5: "clustering", 6: "semantic_similarity",
             7: "code_retrieval"}
    return names.get(int(t), f"task({int(t)})")


class EmbedRuntime:
    """ggufembed.Runtime (api.go:17-36) on one GPU: weights in HBM, the
    reference tokenizer on the host, every call one batched forward per
    requested dimension."""

    def __init__(self, ctx: Context, model: Model, tokenizer: Tokenizer, owns_ctx: bool = False):
        self.ctx, self.model, self.tokenizer = ctx, model, tokenizer
        self._owns_ctx = owns_ctx

    def close(self):
        self.model.close()
        self.tokenizer.close()
        if self._owns_ctx:
            self.ctx.close()

    def embed_dim(self) -> int:
        """EmbedDim (api.go:302-305): the model's full width."""
        return self.model.embed_dim

    def max_seq_len(self) -> int:
        return self.model.max_seq_len

    # ctx (every method): the reference's context.Context argument, see
    # _check_ctx; a cancelled ctx raises Cancelled before the next tokenize or
    # forward starts (work already on the GPU completes).

    def embed(self, texts, ctx=None):
        """Embed (api.go:142-158): TaskSearchQuery prompts, DefaultEmbedDim."""
        if len(texts) == 0:
            return None
        return self.embed_inputs([EmbedInput(Task.SEARCH_QUERY, t, dim=512) for t in texts], ctx)

    def embed_single(self, text: str, ctx=None):
        """EmbedSingle (api.go:160-166)."""
        return self.embed_single_input(EmbedInput(Task.SEARCH_QUERY, text, dim=512), ctx)

    def embed_single_input(self, inp: EmbedInput, ctx=None):
        """EmbedSingleInput (api.go:189-209): the context is checked first."""
        _check_ctx(ctx)
        return self._embed([build_prompt(inp)], [resolve_dim(inp.dim)], ctx)[0]

    def embed_inputs(self, inputs, ctx=None):
        """EmbedInputs (api.go:168-187)."""
        if len(inputs) == 0:
            return None
        prompts, dims = [], []
        for i, inp in enumerate(inputs):
            try:
                prompts.append(build_prompt(inp))
            except EmbedError as e:
                raise EmbedError(f"build prompt for input {i}: {e}") from None
            try:
                dims.append(resolve_dim(inp.dim))
            except ValueError as e:
                raise EmbedError(f"input {i}: {e}") from None
        return self._embed(prompts, dims, ctx)

    def _embed(self, prompts, dims, ctx=None):
        """embedPrompt's checks (api.go:211-234) for every prompt, then one
        packed forward per distinct dimension; results in input order.  The
        context is checked before tokenizing and before each forward (the
        reference checks it before each prompt)."""
        _check_ctx(ctx)
        ids, off = self.tokenizer.encode_batch(prompts)
        max_len = self.model.max_seq_len
        for i in range(len(prompts)):
            n = int(off[i + 1] - off[i])
            if n > max_len:
                raise EmbedError(f"sequence too long: {n} > {max_len}")
        out = [None] * len(prompts)
        for d in sorted(set(dims), reverse=True):
            sel = [i for i, di in enumerate(dims) if di == d]
            seqs = [ids[off[i]:off[i + 1]] for i in sel]
            sub_off = np.zeros(len(sel) + 1, np.int32)
            sub_off[1:] = np.cumsum([len(s) for s in seqs])
            toks = np.concatenate(seqs).astype(np.int32) if sub_off[-1] else np.zeros(1, np.int32)
            _check_ctx(ctx)
            try:
                emb = self.model.forward_packed(toks, sub_off, d)
            except _lib.SemanticaError as e:
                raise EmbedError(f"forward: {e.args[1] if len(e.args) > 1 else e}") from None
            for k, i in enumerate(sel):
                out[i] = emb[k]
        return out


def open_bytes(image: bytes, device: int = 0) -> EmbedRuntime:
    """OpenBytes (api.go:102-106): model and tokenizer from one GGUF image."""
    ctx = Context(device)
    return EmbedRuntime(ctx, Model.from_gguf(ctx, image), Tokenizer.from_gguf(image), owns_ctx=True)


def open(path, device: int = 0) -> EmbedRuntime:  # noqa: A001  (mirrors ggufembed.Open)
    """Open (api.go:94-100)."""
    ctx = Context(device)
    p = os.fspath(path)
    return EmbedRuntime(ctx, Model.from_gguf(ctx, p), Tokenizer.from_gguf(p), owns_ctx=True)
