"""Tokenizers for the server and incremental detokenization.

* ``load_tokenizer(model_path)`` -- a checkpoint's own HF tokenizer (local
  files only) and its stop ids, chosen as the reference's server does
  (server.py:235-276): ``eos_token_id``, every additional special token and
  ``<|im_end|>`` when the vocabulary has it.
* ``SyntheticTokenizer`` -- for random-weight models (no checkpoint):
  ids 0..255 are UTF-8 bytes, the last id of the vocabulary is the stop
  token, every other id decodes to the piece `` w<id>``, so every sampled id
  shows up as text on the wire.  Its chat template is a plain
  ``<|role|>\\ncontent\\n`` transcript ending in ``<|assistant|>\\n``.
* ``IncrementalDetokenizer`` -- the text delta each new id adds.  The
  reference re-decodes the whole output per token and sends
  ``full[len(prev):]`` (server.py:211-223); here only a sliding window of
  ids is re-decoded: text is emitted once the window's decoding grows and
  does not end in U+FFFD (an incomplete UTF-8 sequence or merge), and the
  window then advances.  For byte-level and SentencePiece vocabularies the
  concatenated deltas equal the whole output's decoding.
"""

from __future__ import annotations


class SyntheticTokenizer:
    def __init__(self, vocab_size: int):
        if vocab_size < 258:
            raise ValueError("vocab_size must leave room for 256 byte ids and a stop id")
        self.vocab_size = vocab_size
        self.eos_token_id = vocab_size - 1
        self.unk_token_id = None

    def apply_chat_template(self, messages, tokenize: bool = False, add_generation_prompt: bool = True):
        text = "".join(f"<|{m['role']}|>\n{m['content']}\n" for m in messages)
        if add_generation_prompt:
            text += "<|assistant|>\n"
        return self.encode(text) if tokenize else text

    def encode(self, text: str) -> list[int]:
        return list(text.encode("utf-8"))

    def decode(self, ids, skip_special_tokens: bool = True) -> str:
        out = bytearray()
        for i in ids:
            i = int(i)
            if i < 256:
                out.append(i)
            elif i == self.eos_token_id:
                if not skip_special_tokens:
                    out += b"<|end|>"
            else:
                out += b" w%d" % i
        return out.decode("utf-8", errors="replace")


def stop_ids(tokenizer) -> set[int]:
    """Stop ids of a tokenizer (server.py:256-264)."""
    ids: set[int] = set()
    if getattr(tokenizer, "eos_token_id", None) is not None:
        ids.add(int(tokenizer.eos_token_id))
    ids.update(int(x) for x in getattr(tokenizer, "additional_special_tokens_ids", None) or [])
    convert = getattr(tokenizer, "convert_tokens_to_ids", None)
    if convert is not None:
        im_end = convert("<|im_end|>")
        if isinstance(im_end, int) and im_end != getattr(tokenizer, "unk_token_id", None):
            ids.add(im_end)
    return ids


def load_tokenizer(model_path: str):
    from transformers import AutoTokenizer

    return AutoTokenizer.from_pretrained(model_path, local_files_only=True)


class IncrementalDetokenizer:
    def __init__(self, tokenizer, skip_special_tokens: bool = True):
        self.tok = tokenizer
        self.skip = skip_special_tokens
        self.ids: list[int] = []
        self.prefix = 0     # window start: ids before it are already final text
        self.read = 0       # ids before this index have been emitted

    def _text(self, a: int, b: int) -> str:
        return self.tok.decode(self.ids[a:b], skip_special_tokens=self.skip)

    def push(self, token_id: int) -> str:
        """Text added by ``token_id`` ('' while it is held back)."""
        self.ids.append(int(token_id))
        done = self._text(self.prefix, self.read)
        full = self._text(self.prefix, len(self.ids))
        if len(full) > len(done) and not full.endswith("\ufffd"):
            delta = full[len(done):]
            self.prefix, self.read = self.read, len(self.ids)
            return delta
        return ""

    def flush(self) -> str:
        """Whatever is still held back (e.g. a trailing incomplete sequence)."""
        done = self._text(self.prefix, self.read)
        full = self._text(self.prefix, len(self.ids))
        self.prefix = self.read = len(self.ids)
        return full[len(done):]

    def text(self) -> str:
        return self.tok.decode(self.ids, skip_special_tokens=self.skip)
