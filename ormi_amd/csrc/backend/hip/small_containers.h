// Containers for the scheduler's graph walks. A realize walks a handful of
// nodes (a fused region rarely has more than a dozen), so these keep their
// elements inline and search them linearly, and move to the heap only past
// their inline capacity. The hash sets and vectors they replace made one or
// more allocations per visited node, which dominated the host cost of a
// repeated realize.
#pragma once
#include <cstddef>
#include <memory>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace ormi::hip {
    // A stack (or append-only list) of T with N elements inline.
    template <class T, size_t N>
    class SmallVec {
    public:
        SmallVec() = default;
        SmallVec(const SmallVec&) = delete;
        SmallVec& operator=(const SmallVec&) = delete;

        void push_back(const T& v) {
            if (spill_.empty() && n_ < N) {
                inline_[n_++] = v;
                return;
            }
            if (spill_.empty()) spill_.assign(inline_, inline_ + n_);
            spill_.push_back(v);
            ++n_;
        }
        void pop_back() {
            --n_;
            if (!spill_.empty()) spill_.pop_back();
        }
        T& back() { return spill_.empty() ? inline_[n_ - 1] : spill_.back(); }
        T& operator[](size_t i) { return spill_.empty() ? inline_[i] : spill_[i]; }
        const T& operator[](size_t i) const { return spill_.empty() ? inline_[i] : spill_[i]; }
        size_t size() const { return n_; }
        bool empty() const { return n_ == 0; }

    private:
        T inline_[N]{};
        size_t n_ = 0;
        std::vector<T> spill_;  // every element once past N
    };

    // A map from node address to V: linear search over N inline entries, a
    // hash map beyond.
    template <class K, class V, size_t N = 32>
    class SmallMap {
    public:
        SmallMap() = default;
        SmallMap(const SmallMap&) = delete;
        SmallMap& operator=(const SmallMap&) = delete;

        // The value for k, or nullptr.
        V* find(const K* k) {
            if (big_) {
                auto it = big_->find(k);
                return it == big_->end() ? nullptr : &it->second;
            }
            for (size_t i = 0; i < n_; ++i)
                if (keys_[i] == k) return &vals_[i];
            return nullptr;
        }
        // Inserts (k, v) unless k is present; true when inserted.
        bool insert(const K* k, const V& v) {
            if (find(k)) return false;
            if (!big_ && n_ < N) {
                keys_[n_] = k;
                vals_[n_++] = v;
                return true;
            }
            if (!big_) {
                big_ = std::make_unique<std::unordered_map<const K*, V>>();
                for (size_t i = 0; i < n_; ++i) big_->emplace(keys_[i], vals_[i]);
            }
            big_->emplace(k, v);
            return true;
        }
        void set(const K* k, const V& v) {
            if (V* p = find(k)) *p = v;
            else insert(k, v);
        }
        // Removes k if present.
        void erase(const K* k) {
            if (big_) {
                big_->erase(k);
                return;
            }
            for (size_t i = 0; i < n_; ++i)
                if (keys_[i] == k) {
                    keys_[i] = keys_[n_ - 1];
                    vals_[i] = vals_[n_ - 1];
                    --n_;
                    return;
                }
        }

    private:
        const K* keys_[N]{};
        V vals_[N]{};
        size_t n_ = 0;
        std::unique_ptr<std::unordered_map<const K*, V>> big_;
    };

    // A set of node addresses, as SmallMap without values.
    template <class K, size_t N = 32>
    class SmallSet {
    public:
        SmallSet() = default;
        SmallSet(const SmallSet&) = delete;
        SmallSet& operator=(const SmallSet&) = delete;

        bool contains(const K* k) const {
            if (big_) return big_->count(k) > 0;
            for (size_t i = 0; i < n_; ++i)
                if (keys_[i] == k) return true;
            return false;
        }
        // True when k was not present.
        bool insert(const K* k) {
            if (contains(k)) return false;
            if (!big_ && n_ < N) {
                keys_[n_++] = k;
                return true;
            }
            if (!big_) big_ = std::make_unique<std::unordered_set<const K*>>(keys_, keys_ + n_);
            big_->insert(k);
            return true;
        }
        void erase(const K* k) {
            if (big_) {
                big_->erase(k);
                return;
            }
            for (size_t i = 0; i < n_; ++i)
                if (keys_[i] == k) {
                    keys_[i] = keys_[--n_];
                    return;
                }
        }

    private:
        const K* keys_[N]{};
        size_t n_ = 0;
        std::unique_ptr<std::unordered_set<const K*>> big_;
    };
}
