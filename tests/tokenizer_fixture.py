"""A small byte-level BPE tokenizer.json written with the `tokenizers`
library (test infrastructure).  It has the shape of the Llama 3 tokenizer:
byte-level pre-tokenizer and decoder, BOS added by a template post-processor
when special tokens are requested, BOS / EOS as the first two ids."""
from __future__ import annotations

CORPUS = [
    "The capital of France is Paris. The capital of Germany is Berlin.",
    "A quick brown fox jumps over the lazy dog; the dog sleeps.",
    "Perplexity measures how well a model predicts a sample of text.",
    "Matrix cores multiply tiles of int8 values and accumulate in int32.",
    "Tokens stream out one by one, each decoded as soon as it is sampled.",
] * 8

BOS, EOS = "<|begin_of_text|>", "<|end_of_text|>"


def write_tokenizer(path: str, vocab_size: int = 400) -> tuple[int, int]:
    """Trains the tokenizer on CORPUS and saves it; returns (bos_id, eos_id)."""
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, processors, trainers
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, special_tokens=[BOS, EOS],
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet(), show_progress=False)
    tok.train_from_iterator(CORPUS, trainer)
    bos, eos = tok.token_to_id(BOS), tok.token_to_id(EOS)
    tok.post_processor = processors.TemplateProcessing(single=f"{BOS} $A", special_tokens=[(BOS, bos)])
    tok.save(path)
    return bos, eos
