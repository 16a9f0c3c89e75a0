"""Text <-> token ids for the scheduler, over a Hugging Face tokenizer read from
the model directory (litelang/scheduler/tokenizer/tokenizer.py:4-31): left
padding, the tokenizer's eos id, batch encode with padding and truncation,
encode_single returning a batch of one sequence, decode skipping special
tokens without clean-up of tokenisation spaces. Only local files are read.
"""
from __future__ import annotations


class Tokenizer:
    def __init__(self, model_path: str):
        from transformers import AutoTokenizer
        self.tokenizer = AutoTokenizer.from_pretrained(model_path, local_files_only=True)
        self.tokenizer.padding_side = "left"
        self.eos_token_id = self.tokenizer.eos_token_id

    def encode(self, prompts):
        """(input_ids, attention_mask) of a left-padded batch (tokenizer.py:10-14)."""
        t = self.tokenizer(prompts, return_tensors="pt", padding=True, truncation=True)
        return t["input_ids"], t["attention_mask"]

    def encode_single(self, prompt):
        """input_ids [1, n] of one prompt (tokenizer.py:16-24)."""
        t = self.tokenizer([prompt], return_tensors="pt", padding=True, truncation=True)
        return t["input_ids"]

    def decode(self, generate_ids):
        """One string per sequence of ids (tokenizer.py:26-30)."""
        return self.tokenizer.batch_decode(generate_ids, skip_special_tokens=True,
                                           clean_up_tokenization_spaces=False)
