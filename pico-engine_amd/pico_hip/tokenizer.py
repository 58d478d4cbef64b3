"""GPT-2 style byte-level BPE rebuilt from GGUF tokenizer metadata (host only).

Same surface as the reference's tokenizer.py (``BPETokenizer``, ``from_gguf``, :40-124):
vocabulary ``tokenizer.ggml.tokens``, merge ranks ``tokenizer.ggml.merges``, bos/eos ids
(default -1), ``<|...|>`` specials matched whole before BPE, bytes mapped to printable symbols
with the standard GPT-2 table. Not on the timed path (benchmarks feed token ids directly).
"""

from __future__ import annotations

import regex as re


def byte_symbols() -> dict[int, str]:
    """GPT-2 byte -> printable-unicode map (bytes outside the printable set go to 256+)."""
    printable = (list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) +
                 list(range(0xAE, 0x100)))
    table, extra = {}, 0
    for b in range(256):
        if b in printable:
            table[b] = chr(b)
        else:
            table[b] = chr(256 + extra)
            extra += 1
    return table


_B2U = byte_symbols()
_U2B = {u: b for b, u in _B2U.items()}
_PRETOKENIZE = re.compile(
    r"""'(?:[sdmt]|ll|ve|re)| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+""")
_SPECIAL = re.compile(r"<\|[^|]*\|>")


class BPETokenizer:
    def __init__(self, vocab: list[str], merges: list[str], bos_id: int, eos_id: int):
        self.vocab = list(vocab)
        self.vocab_id = {tok: i for i, tok in enumerate(self.vocab)}
        self.ranks = {m: r for r, m in enumerate(merges)}
        self.bos_id, self.eos_id = bos_id, eos_id
        specials = sorted((t for t in self.vocab if _SPECIAL.fullmatch(t)), key=len, reverse=True)
        self.special_set = set(specials)
        self._split_special = re.compile("(" + "|".join(re.escape(s) for s in specials) + ")") if specials else None

    @property
    def n_vocab(self) -> int:
        return len(self.vocab)

    def _merge(self, symbols: list[str]) -> list[str]:
        while len(symbols) > 1:
            ranked = [(self.ranks.get(symbols[i] + " " + symbols[i + 1]), i) for i in range(len(symbols) - 1)]
            ranked = [(r, i) for r, i in ranked if r is not None]
            if not ranked:
                break
            _, i = min(ranked)
            symbols = symbols[:i] + [symbols[i] + symbols[i + 1]] + symbols[i + 2:]
        return symbols

    def _encode_plain(self, text: str) -> list[int]:
        ids: list[int] = []
        for piece in _PRETOKENIZE.findall(text):
            mapped = "".join(_B2U[b] for b in piece.encode("utf-8"))
            for sym in self._merge(list(mapped)):
                if sym in self.vocab_id:
                    ids.append(self.vocab_id[sym])
                else:  # unknown merge result: fall back to single-byte symbols
                    ids.extend(self.vocab_id[c] for c in sym)
        return ids

    def encode(self, text: str) -> list[int]:
        if self._split_special is None:
            return self._encode_plain(text)
        ids: list[int] = []
        for part in self._split_special.split(text):
            if part in self.special_set:
                ids.append(self.vocab_id[part])
            elif part:
                ids.extend(self._encode_plain(part))
        return ids

    def decode(self, ids: list[int]) -> str:
        text = "".join(self.vocab[i] for i in ids)
        return bytes(_U2B[c] for c in text if c in _U2B).decode("utf-8", errors="replace")


def from_gguf(metadata: dict) -> BPETokenizer:
    model = metadata.get("tokenizer.ggml.model", "")
    if model != "gpt2":
        raise ValueError(f"unsupported tokenizer model {model!r} (only gpt2 byte-level BPE)")
    return BPETokenizer(metadata["tokenizer.ggml.tokens"], metadata.get("tokenizer.ggml.merges", []),
                        int(metadata.get("tokenizer.ggml.bos_token_id", -1)),
                        int(metadata.get("tokenizer.ggml.eos_token_id", -1)))
