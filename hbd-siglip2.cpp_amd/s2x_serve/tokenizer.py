"""SentencePiece tokenization as the reference's Tokenizer::encode
(src/siglip2_tokenizer.cpp:52-93): the pieces' ids, then EOS; padded with
the pad id (0 where the model defines none, the SigLIP2 / Gemma
convention) to max_length, the mask 1 on kept tokens; on truncation EOS
stays in the last position.  max_length <= 0: natural length, no padding.
"""


class Tokenizer:
    def __init__(self, model_path):
        import sentencepiece
        self.sp = sentencepiece.SentencePieceProcessor(model_file=str(model_path))
        self.eos_id = self.sp.eos_id()
        pad = self.sp.pad_id()
        self.pad_id = pad if pad >= 0 else 0

    @property
    def vocab_size(self):
        return self.sp.get_piece_size()

    def encode(self, text, max_length):
        ids = list(self.sp.encode(text))
        if self.eos_id >= 0:
            ids.append(self.eos_id)
        if max_length <= 0:
            return ids, [1] * len(ids)
        out = [self.pad_id] * max_length
        mask = [0] * max_length
        keep = min(len(ids), max_length)
        out[:keep] = ids[:keep]
        mask[:keep] = [1] * keep
        if self.eos_id >= 0 and len(ids) > max_length:
            out[max_length - 1] = self.eos_id
        return out, mask
